"""Loaders and ctypes binders for the kernel libraries.

Counterpart of the reference's ``frame_analytics/_cabi.py`` (load_cuda at
_cabi.py:515, load_cpu at :474-512, the binders at :414-462, _check_abi at
:465-471): find a library (building it in-tree if it is missing), bind the
prototypes of ``include/fa_abi.h`` / ``include/fa_cpu_abi.h`` and reject a
library whose ABI version does not match this Python package.

Unlike the reference there is no prebuilt/JIT cache directory and no
baseline/AVX2 pair of CPU builds: ``libfa_gpu.so`` (gfx950) and
``libfa_cpu.so`` (x86-64 AVX2 + FMA, used only where the CPU has both) sit next
to this file.
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
          _P, _P, _P, _I, _I, _P], _I),
    "fa_gpu_gmsd_ex":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _D, _D, _I, _P, _P, _P, _I, _P, _P, _I, _P],
         _I),
    "fa_gpu_gmsd_backward":
        ([_P, _P, _I, _I, _I, _I, _I, _D, _D, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ms_ssim_reduce": ([_P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ms_ssim_head": ([_P, _I, _I, _I, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ms_ssim_head_backward": ([_P, _I, _I, _I, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_noalloc":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P, _P, _I, _P], _I),
    "fa_gpu_pixel_reduce_once":
        ([_P, _P, _I, _L, _L, _I, _D, _D, _P, _I, _P, _P, _P, _P, _P, _I, _P], _I),
    "fa_gpu_gmsd_once":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _D, _D, _I, _P, _P, _I, _P, _P, _P, _P, _I,
          _P], _I),
    "fa_gpu_ssim_once":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _D, _D, _D, _P, _P, _I, _P, _P, _P,
          _I, _P], _I),
    "fa_gpu_ms_ssim_workspace": ([_I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "fa_gpu_ms_ssim":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _D, _D, _D, _P, _I, _P, _L, _P, _P,
          _P, _I, _P], _I),
    "fa_gpu_ssim_cs_coef":
        ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _I, _P, _P, _I, _P, _P, _P, _P, _I, _P,
          _I, _I, _P], _I),
    "fa_gpu_ssim_cs_scatter":
        ([_P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _D, _P, _I, _P, _P, _I, _P, _P, _I, _P], _I),
    "fa_gpu_ssim_cs_backward_ex":
        ([_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _D, _D, _D, _P, _P, _I, _P, _P, _P,
          _I, _P], _I),
}


# one line per entry point of include/fa_cpu_abi.h (reference _cabi.py:416-423)
CPU_SIGNATURES = {
    "fa_cpu_abi_version": ([], _I),
    "fa_cpu_has_avx2": ([], _I),
    "fa_cpu_set_num_threads": ([_I], _I),
    "fa_cpu_num_threads": ([], _I),
    "fa_cpu_pixel_reduce": ([_P, _P, _I, _L, _L, _I, _D, _D, _I, _P], _I),
    "fa_cpu_ssim": ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P], _I),
    "fa_cpu_ssim_cs": ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P], _I),
    "fa_cpu_gmsd": ([_P, _P, _I, _I, _I, _I, _I, _D, _D, _I, _P, _P], _I),
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


def bind(lib: ctypes.CDLL, signatures: Optional[dict] = None) -> ctypes.CDLL:
    for name, (args, res) in (SIGNATURES if signatures is None else signatures).items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _check_abi(lib: ctypes.CDLL, origin: Path, cpu: bool = False) -> None:
    got = lib.fa_cpu_abi_version() if cpu else lib.fa_gpu_abi_version()
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


def load_cpu(path: Optional[Path] = None) -> Tuple[Optional[ctypes.CDLL], str]:
    """Return ``(lib, origin)`` for the host kernel library, or ``(None,
    reason)`` when this CPU lacks AVX2 + FMA (the library's hot loops are
    compiled for them; ``fa_cpu_has_avx2`` itself is safe to call anywhere).
    Built in-tree with the host compiler when missing."""
    p = Path(path) if path is not None else _build.cpu_library_path()
    origin = "in-tree"
    if not p.exists():
        _build.build_cpu(verbose=_verbose())
        origin = "built"
    lib = bind(ctypes.CDLL(str(p)), CPU_SIGNATURES)
    _check_abi(lib, p, cpu=True)
    if not lib.fa_cpu_has_avx2():
        return None, "host CPU lacks AVX2/FMA"
    return lib, origin
