"""Loader and ctypes binder for the gfx950 kernel library.

Counterpart of the reference's ``frame_analytics/_cabi.py`` (load_cuda at
_cabi.py:515, _bind_cuda at :432-462, _check_abi at :465-471): find the
library (building it in-tree with hipcc if it is missing), bind the
prototypes of ``include/fa_abi.h`` and reject a library whose ABI version does
not match this Python package.

Unlike the reference there is no prebuilt/JIT cache directory and no CPU
library: the only native code is ``libfa_gpu.so`` next to this file.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

from . import _build

FA_ABI_VERSION = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_D = ctypes.c_double

# name -> (argtypes, restype); one line per entry point of include/fa_abi.h
SIGNATURES = {
    "fa_gpu_abi_version": ([], _I),
    "fa_gpu_error_string": ([_I], ctypes.c_char_p),
    "fa_gpu_device_count": ([_P], _I),
    "fa_gpu_pixel_workspace": ([_L, _L, _I, _P], _I),
    "fa_gpu_pixel_reduce":
        ([_P, _P, _I, _L, _L, _I, _D, _D, _P, _I, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_workspace": ([_I, _I, _I, _P], _I),
    "fa_gpu_ssim":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P, _I, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_cs":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P, _I, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_backward":
        ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _D, _D, _D, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_cs_backward":
        ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _D, _D, _D, _P, _P, _P, _I, _P], _I),
    "fa_gpu_gmsd_workspace": ([_I, _I, _I, _P], _I),
    "fa_gpu_gmsd":
        ([_P, _P, _I, _I, _I, _I, _I, _D, _D, _I, _P, _P, _I, _P, _P, _I, _P], _I),
    # extensions without a reference counterpart
    "fa_gpu_pixel_reduce_ex":
        ([_P, _P, _I, _L, _I, _I, _I, _P, _P, _P, _I, _D, _D, _P, _I, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_ex":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _D, _D, _D, _P, _P, _I, _P, _P,
          _I, _P], _I),
    "fa_gpu_ssim_cs_ex":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _D, _D, _D, _P, _P, _I, _P, _P,
          _P, _P, _I, _I, _P], _I),
    "fa_gpu_gmsd_ex":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _D, _D, _I, _P, _P, _P, _I, _P, _P, _I, _P],
         _I),
    "fa_gpu_gmsd_backward":
        ([_P, _P, _I, _I, _I, _I, _I, _D, _D, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ms_ssim_combine": ([_P, _P, _I, _I, _I, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_cs_backward_ex":
        ([_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _D, _D, _D, _P, _P, _I, _P, _P, _P,
          _I, _P], _I),
}


class KernelError(RuntimeError):
    """A native entry point returned a non-zero status."""


def status_text(code: int, lib=None) -> str:
    if lib is not None:
        try:
            msg = lib.fa_gpu_error_string(int(code))
            if msg:
                return f"status {code}: {msg.decode(errors='replace')}"
        except Exception:
            pass
    return f"status {code}"


def _verbose() -> bool:
    return os.environ.get("FA_VERBOSE", "0") == "1"


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _check_abi(lib: ctypes.CDLL, origin: Path) -> None:
    got = lib.fa_gpu_abi_version()
    if got != FA_ABI_VERSION:
        raise RuntimeError(
            f"{origin} reports ABI version {got}, this package expects "
            f"{FA_ABI_VERSION}; rebuild it (python -m frame_analytics_amd._build)")


def load_gpu(path: Optional[Path] = None) -> Tuple[ctypes.CDLL, str]:
    """Return ``(lib, origin)``; ``origin`` is ``"in-tree"`` or ``"built"``.

    The library is only built here when it is missing: a stale-but-present
    build is used as is (``__graft_entry__.build()`` / ``_build.build()`` is the
    explicit rebuild), so a GPU run never recompiles behind the caller's back.
    """
    p = Path(path) if path is not None else _build.library_path()
    origin = "in-tree"
    if not p.exists():
        _build.build(verbose=_verbose())
        origin = "built"
    # RTLD_GLOBAL is not needed: nothing links against this library.
    lib = bind(ctypes.CDLL(str(p)))
    _check_abi(lib, p)
    return lib, origin
