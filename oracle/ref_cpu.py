"""ctypes binding of the reference's own CPU kernels -- TEST INFRASTRUCTURE ONLY.

``oracle/_ref/libfa_cpu_ref.so`` is compiled by ``oracle/Makefile`` from the
reference's ``frame_analytics/csrc/fa_cpu.cpp`` (where it lies under
/root/reference); it travels to the GPU box as a built file.  It serves two
purposes: the ``cpu_baseline`` leg of ``bench.py`` (kind "reference"), and an
independent float32 implementation against which tests pin
``oracle/reference.py`` at the reference's own 5e-6 gate.

The entry points and their argument conventions are those of the reference's
C ABI (reference fa_abi.h:77-115).
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_ref" / "libfa_cpu_ref.so"
PSNR_NONE = -1.0e300
OP = {"mse": 0, "l1": 1, "charbonnier": 2, "huber": 3}
DTYPE = {np.dtype(np.uint8): 0, np.dtype(np.float32): 3, np.dtype(np.float64): 4}

_P, _I, _L, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
_SIG = {
    "fa_cpu_abi_version": ([], _I),
    "fa_cpu_has_avx2": ([], _I),
    "fa_cpu_set_num_threads": ([_I], _I),
    "fa_cpu_num_threads": ([], _I),
    "fa_cpu_pixel_reduce": ([_P, _P, _I, _L, _L, _I, _D, _D, _I, _P], _I),
    "fa_cpu_ssim": ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P], _I),
    "fa_cpu_ssim_cs": ([_P, _P, _I, _I, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P], _I),
    "fa_cpu_gmsd": ([_P, _P, _I, _I, _I, _I, _I, _D, _D, _I, _P, _P], _I),
}

_lib = None


def available() -> bool:
    return LIB_PATH.exists()


def load(threads: Optional[int] = None):
    """Load the library; ``threads`` sizes its pool (first call only)."""
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIG.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        if threads:
            lib.fa_cpu_set_num_threads(int(threads))
        _lib = lib
    return _lib


def _c(a):
    a = np.ascontiguousarray(a)
    return a, a.ctypes.data


def _check(rc):
    if rc != 0:
        raise RuntimeError(f"reference CPU kernel returned status {rc}")


def pixel_reduce(x, y, op="mse", param=0.0, psnr_bias=PSNR_NONE, per_image=False):
    lib = load()
    x, px = _c(x)
    y, py = _c(y)
    n = x.shape[0]
    out = np.zeros(n if per_image else 1, np.float64)
    _check(lib.fa_cpu_pixel_reduce(px, py, DTYPE[x.dtype], n, x.size // n, OP[op],
                                   float(param), float(psnr_bias), int(per_image),
                                   out.ctypes.data))
    return out if per_image else float(out[0])


def _window(win_size, sigma):
    c = np.arange(win_size, dtype=np.float64) - (win_size - 1) / 2.0
    g = np.exp(-(c * c) / (2.0 * sigma * sigma))
    return np.ascontiguousarray((g / g.sum()).astype(np.float32))


def ssim_per_image(x, y, data_range=255.0, win_size=11, sigma=1.5, K=(0.01, 0.03)):
    """Per-image SSIM means from the reference CPU kernel (plane sums folded
    per image as reference backend.py:517-523 does)."""
    lib = load()
    x, px = _c(x)
    y, py = _c(y)
    n, c, h, w = x.shape
    win = _window(win_size, sigma)
    per_plane = np.zeros(n * c, np.float64)
    L = float(data_range)
    _check(lib.fa_cpu_ssim(px, py, DTYPE[x.dtype], n, c, h, w, win.ctypes.data, win_size,
                           0.5 * L, (K[0] * L) ** 2, (K[1] * L) ** 2, None,
                           per_plane.ctypes.data))
    npix = (h - win_size + 1) * (w - win_size + 1)
    return per_plane.reshape(n, c).sum(axis=1) / (npix * c)


def ssim_cs(x, y, data_range=255.0, win_size=11, sigma=1.5, K=(0.01, 0.03)):
    lib = load()
    x, px = _c(x)
    y, py = _c(y)
    n, c, h, w = x.shape
    win = _window(win_size, sigma)
    s = np.zeros(n * c, np.float64)
    cs = np.zeros(n * c, np.float64)
    L = float(data_range)
    _check(lib.fa_cpu_ssim_cs(px, py, DTYPE[x.dtype], n, c, h, w, win.ctypes.data, win_size,
                              0.5 * L, (K[0] * L) ** 2, (K[1] * L) ** 2, s.ctypes.data,
                              cs.ctypes.data))
    return s.reshape(n, c), cs.reshape(n, c)


def gmsd(x, y, data_range=255.0, downsample=True):
    lib = load()
    x, px = _c(x)
    y, py = _c(y)
    n, c, h, w = x.shape
    L = float(data_range)
    mean = np.zeros(n, np.float64)
    std = np.zeros(n, np.float64)
    _check(lib.fa_cpu_gmsd(px, py, DTYPE[x.dtype], n, c, h, w, 170.0 * (L / 255.0) ** 2,
                           (1e-6 * L) ** 2, int(downsample), mean.ctypes.data, std.ctypes.data))
    return mean, std
