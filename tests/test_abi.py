"""The C-ABI libraries: build, load, export exactly what include/fa_abi.h
(libfa_gpu.so) and include/fa_cpu_abi.h (libfa_cpu.so) declare, with the
ctypes prototypes the binders use.  No GPU compute calls (these run without a
GPU); the status and workspace queries used here are pure host arithmetic.
The host library's compute is covered by tests/test_cpu_kernels.py."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from frame_analytics_amd import _build, _cabi

HEADER = Path(__file__).resolve().parents[1] / "include" / "fa_abi.h"
CPU_HEADER = HEADER.with_name("fa_cpu_abi.h")


def _declared(header: Path = HEADER):
    """name -> number of parameters, for every FA_API function in the header."""
    txt = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"FA_API\s+[\w\s\*]+?\b(fa_\w+)\s*\(([^)]*)\)\s*;", txt, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    path = _build.library_path()
    if not path.exists():
        _build.build()
    return _cabi.bind(ctypes.CDLL(str(path)))


def test_header_and_binder_agree():
    decl = _declared()
    assert len(decl) == 29  # 12 reference entry points + 17 extensions
    assert set(decl) == set(_cabi.SIGNATURES)
    for name, n in decl.items():
        assert len(_cabi.SIGNATURES[name][0]) == n, name


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_cpu_header_and_binder_agree():
    decl = _declared(CPU_HEADER)
    assert len(decl) == 8  # the reference's eight fa_cpu_* entry points
    assert set(decl) == set(_cabi.CPU_SIGNATURES)
    for name, n in decl.items():
        assert len(_cabi.CPU_SIGNATURES[name][0]) == n, name


def test_cpu_library_exports_every_declared_symbol():
    path = _build.cpu_library_path()
    if not path.exists():
        _build.build_cpu()
    lib = _cabi.bind(ctypes.CDLL(str(path)), _cabi.CPU_SIGNATURES)
    for name in _declared(CPU_HEADER):
        assert hasattr(lib, name), name
    assert lib.fa_cpu_abi_version() == _cabi.FA_ABI_VERSION
    # nothing but the declared entry points is exported
    nm = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True,
                        text=True)
    if nm.returncode == 0:
        exported = {ln.split()[-1] for ln in nm.stdout.splitlines()
                    if " T " in ln and ln.split()[-1].startswith("fa_")}
        assert exported == set(_declared(CPU_HEADER))


def test_abi_version_and_status_strings(lib):
    assert lib.fa_gpu_abi_version() == _cabi.FA_ABI_VERSION
    assert lib.fa_gpu_error_string(0) == b"ok"
    assert lib.fa_gpu_error_string(3) == b"unsupported window size"
    assert b"GPU" in lib.fa_gpu_error_string(7)


def test_workspace_queries(lib):
    out = ctypes.c_int(0)
    assert lib.fa_gpu_ssim_workspace(1080, 1920, 11, ctypes.byref(out)) == 0
    # 246 output columns per 256-lane strip; slots for the smallest row tile (4)
    assert out.value == 8 * 268
    assert lib.fa_gpu_ssim_workspace(8, 8, 11, ctypes.byref(out)) == 2  # FA_E_SHAPE
    assert lib.fa_gpu_ssim_workspace(64, 64, 4, ctypes.byref(out)) == 3  # even window
    assert lib.fa_gpu_ssim_workspace(64, 64, 13, ctypes.byref(out)) == 3
    assert lib.fa_gpu_ssim_workspace(64, 64, 11, None) == 5  # FA_E_ARG
    assert lib.fa_gpu_gmsd_workspace(1080, 1920, 1, ctypes.byref(out)) == 0
    assert out.value == 16 * 135  # 538x958 output: 62-column strips, 4-row tiles
    assert lib.fa_gpu_gmsd_workspace(5, 5, 1, ctypes.byref(out)) == 2
    # fa_gpu_ms_ssim's workspace: levels, partial sums and scratch, every scale checked
    nb = ctypes.c_int64(0)
    assert lib.fa_gpu_ms_ssim_workspace(0, 8, 3, 1080, 1920, 11, 5, 0, ctypes.byref(nb)) == 0
    u8 = nb.value
    # at least the float16 first level and the float32 second of both inputs
    assert u8 >= 2 * 24 * (540 * 960 * 2 + 270 * 480 * 4)
    assert lib.fa_gpu_ms_ssim_workspace(3, 8, 3, 1080, 1920, 11, 5, 0, ctypes.byref(nb)) == 0
    assert nb.value > u8  # float64 levels under float32 input
    assert lib.fa_gpu_ms_ssim_workspace(0, 1, 1, 160, 200, 11, 5, 0, ctypes.byref(nb)) == 2
    assert lib.fa_gpu_ms_ssim_workspace(0, 1, 1, 176, 176, 11, 5, 0, ctypes.byref(nb)) == 0
    assert lib.fa_gpu_ms_ssim_workspace(0, 1, 1, 176, 176, 11, 9, 0, ctypes.byref(nb)) == 2
    assert lib.fa_gpu_ms_ssim_workspace(0, 1, 2, 176, 176, 11, 5, 1, ctypes.byref(nb)) == 2


def test_argument_validation_before_any_gpu_work(lib):
    """Null pointers and bad codes are rejected on the host."""
    assert lib.fa_gpu_pixel_reduce(None, None, 0, 1, 16, 0, 0.0, -1e300, None, 1,
                                   None, None, None, None, 0, None) == 5
    one = ctypes.c_double(0)
    p = ctypes.addressof(one)
    assert lib.fa_gpu_pixel_reduce(p, p, 0, 1, 16, 9, 0.0, -1e300, p, 1,
                                   None, None, None, None, 0, None) == 4  # FA_E_OP
    assert lib.fa_gpu_pixel_reduce(p, p, 0, 0, 16, 0, 0.0, -1e300, p, 1,
                                   None, None, None, None, 0, None) == 2
    w5 = (ctypes.c_double * 5)(0.0448, 0.2856, 0.3001, 0.2363, 0.1333)
    ms = lib.fa_gpu_ms_ssim
    # a scale too small, and a workspace too small: refused before any launch
    assert ms(p, p, 0, 1, 1, 160, 200, None, None, None, p, 11, 127.5, 6.5, 58.5, w5, 5, p,
              1 << 40, None, p, None, 0, None) == 2
    assert ms(p, p, 0, 1, 1, 176, 176, None, None, None, p, 11, 127.5, 6.5, 58.5, w5, 5, p,
              16, None, p, None, 0, None) == 5
    assert ms(p, p, 0, 1, 1, 176, 176, None, None, None, p, 11, 127.5, 6.5, 58.5, w5, 5, p,
              1 << 40, p, None, None, 0, None) == 5  # no output
    once = lib.fa_gpu_pixel_reduce_once
    assert once(p, p, 0, 1, 16, 0, 0.0, -1e300, None, 1, p, p, None, None, None, 0, None) == 5
    assert once(p, p, 0, 1, 16, 4, 0.0, -1e300, p, 1, p, p, None, None, None, 0, None) == 4
    assert once(p, p, 0, 70000, 16, 0, 0.0, -1e300, p, 1, p, p, None, None, None, 0,
                None) == 2
    assert lib.fa_gpu_ssim(p, p, 0, 1, 1, 64, 64, p, 12, 0.5, 1e-4, 9e-4, None, p, 1,
                           None, None, 0, None) == 3
    assert lib.fa_gpu_ssim(p, p, 0, 1, 1, 64, 64, p, 11, 0.5, 1e-4, 9e-4, None, p, 99,
                           None, None, 0, None) == 5  # bpp mismatch
    assert lib.fa_gpu_ssim_backward(p, p, None, None, p, 11, 1, 1, 64, 64, 0.5, 1e-4, 9e-4,
                                    p, p, None, 0, None) == 5  # no upstream gradient
    assert lib.fa_gpu_gmsd(p, p, 0, 1, 1, 64, 64, 170.0, 0.0, 1, p, p, 99, p, p, 0, None) == 5
    lw = (ctypes.c_double * 3)(0.299, 0.587, 0.114)
    assert lib.fa_gpu_gmsd_ex(p, p, 0, 1, 1, 64, 64, None, None, lw, 170.0, 0.0, 1, None, p, p,
                              99, p, p, 0, None) == 2  # luma needs 3 channels
    bad = (ctypes.c_int64 * 3)(3 * 64 * 64, 64 * 64, 32)  # rows overlap
    assert lib.fa_gpu_gmsd_backward(p, p, 0, 1, 1, 64, 64, 170.0, 0.0, 1, p, p, None, None, p,
                                    p, None, 0, None) == 1  # uint8 has no gradient
    assert lib.fa_gpu_gmsd_backward(p, p, 3, 1, 1, 64, 64, 170.0, 0.0, 1, p, p, None, None, p,
                                    None, None, 0, None) == 5  # neither dx nor dy
    ptrs = (ctypes.c_void_p * 5)(p, p, p, p, p)
    wts = (ctypes.c_double * 5)(0.0448, 0.2856, 0.3001, 0.2363, 0.1333)
    slots = (ctypes.c_int * 5)(4, 4, 4, 4, 4)
    npix = (ctypes.c_double * 5)(100.0, 50.0, 20.0, 8.0, 2.0)
    red = lib.fa_gpu_ms_ssim_reduce
    assert red(ptrs, slots, npix, wts, 9, 1, 1, p, p, None, 0, None) == 2  # > 8 scales
    assert red(ptrs, slots, npix, wts, 5, 1, 1, p, None, None, 0, None) == 5  # no output
    assert red(ptrs, slots, npix, wts, 5, 1, 1, None, p, None, 0, None) == 5  # no scratch
    zero = (ctypes.c_int * 5)(4, 0, 4, 4, 4)
    assert red(ptrs, zero, npix, wts, 5, 1, 1, p, p, None, 0, None) == 2  # empty scale
    # partial sums left unreduced need the slot count back, and both means go together
    cs2 = (3, 1, 1, 64, 64, None, None, None, p, 11, 0.5, 1e-4, 9e-4, p, p, 99)
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs2, None, None, None, None, None, 4, 0, None) == 5
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs2, p, None, None, None, None, 4, 0, None) == 5
    ws = ctypes.c_int(0)
    assert lib.fa_gpu_gmsd_workspace(64, 64, 1, ctypes.byref(ws)) == 0
    assert lib.fa_gpu_gmsd_ex(p, p, 0, 1, 3, 64, 64, bad, None, None, 170.0, 0.0, 1, None, p,
                              p, ws.value, p, p, 0, None) == 2
    # the fused pyramid step insists on an exact level type
    cs = (1, 1, 1, 64, 64, None, None, None, p, 11, 0.5, 1e-4, 9e-4, p, p, 99, p, p)  # f16
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs, None, p, p, 3, 0, None) == 1  # float16 -> float32
    assert lib.fa_gpu_ssim_cs_ex(p, p, 2, *cs[1:], None, p, p, 3, 0, None) == 1  # bfloat16
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs, None, p, p, 0, 0, None) == 1  # uint8 levels
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs, None, None, p, 4, 0, None) == 5  # one level buffer
    assert lib.fa_gpu_ssim_cs_ex(p, p, *cs, None, p, p, 4, 0, None) == 5  # bpp mismatch
    assert lib.fa_gpu_ssim_cs_ex(p, p, 0, *cs[1:], None, p, p, 3, 0, None) == 5  # u8 -> f32 ok
    lw = (ctypes.c_double * 4)(0.299, 0.587, 0.114, 0.0)
    u8l = (0, 1, 3, 64, 64, None, None, lw, p, 11, 0.5, 1e-4, 9e-4, p, p, 99, p, p)
    assert lib.fa_gpu_ssim_cs_ex(p, p, *u8l, None, p, p, 3, 0, None) == 1  # luma pools to f64
    ws = ctypes.c_int(0)
    assert lib.fa_gpu_ssim_workspace(64, 64, 11, ctypes.byref(ws)) == 0
    one = u8l[:2] + (1,) + u8l[3:15] + (ws.value,) + u8l[16:]
    assert lib.fa_gpu_ssim_cs_ex(p, p, *one, None, None, None, 4, 0, None) == 2  # luma needs 3 channels
    rows = (ctypes.c_int64 * 3)(3 * 64 * 64, 64 * 64, 60)  # rows overlap
    assert lib.fa_gpu_ssim_ex(p, p, 0, 1, 3, 64, 64, rows, None, None, p, 11, 0.5, 1e-4, 9e-4,
                              None, p, 99, None, None, 0, None) == 5  # bpp checked first
    assert lib.fa_gpu_ssim_ex(p, p, 0, 1, 3, 64, 64, rows, None, None, p, 11, 0.5, 1e-4, 9e-4,
                              None, p, ws.value, None, None, 0, None) == 2
    assert lib.fa_gpu_ssim_cs_backward_ex(p, p, 0, p, p, p, 11, 1, 1, 64, 64, 0.5, 1e-4,
                                          9e-4, None, None, 0, p, p, None, 0,
                                          None) == 1  # uint8 input
    assert lib.fa_gpu_ssim_cs_backward_ex(p, p, 3, p, p, p, 11, 1, 1, 64, 64, 0.5, 1e-4,
                                          9e-4, p, None, 1, p, p, None, 0,
                                          None) == 1  # float16 pyramid gradient


def test_noalloc_bounds_its_scratch_on_the_host(lib):
    """fa_gpu_ssim_noalloc rejects a call whose partial sums would not fit its
    fixed scratch (FA_NOALLOC_SLOTS float64) before any HIP call: the checks
    here run without a GPU, with null data pointers."""
    slots = ctypes.c_int(0)
    assert lib.fa_gpu_ssim_workspace(1080, 1920, 11, ctypes.byref(slots)) == 0
    cap = 1 << 20
    planes_max = cap // slots.value
    args = (None, None, 0)
    tail = (None, 11, 127.5, 6.5025, 58.5225, None, None, None, 0, None)
    # one plane more than fits
    assert lib.fa_gpu_ssim_noalloc(*args, planes_max + 1, 1, 1080, 1920, *tail) == 8
    assert lib.fa_gpu_ssim_noalloc(*args, 1, planes_max + 1, 1080, 1920, *tail) == 8
    assert b"scratch" in lib.fa_gpu_error_string(8)
    # shape errors come first, as in fa_gpu_ssim
    assert lib.fa_gpu_ssim_noalloc(*args, 1, 1, 8, 8, *tail) == 2
    assert lib.fa_gpu_ssim_noalloc(*args, 1, 1, 64, 64, None, 12, *tail[2:]) == 3
