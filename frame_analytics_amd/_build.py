"""Builds the gfx950 kernel library ``libfa_gpu.so`` in-tree with hipcc, and
the host kernel library ``libfa_cpu.so`` (``csrc/fa_cpu.cpp``, C ABI in
``include/fa_cpu_abi.h``) with the host C++ compiler.

The library is plain HIP C++ behind the C ABI in ``include/fa_abi.h``; it
links only the HIP runtime, whose soname (``libamdhip64.so.7``) is the one
torch itself loads, so after ``import torch`` the dynamic loader hands both the
same runtime and torch's ``hipStream_t`` handles are valid in the library.

Every ``.hip`` file under ``csrc/`` is compiled to its own object in parallel,
then linked.  ``FA_HIP_ARCHS`` overrides the target list (default ``gfx950``).
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
from pathlib import Path
from typing import List, Sequence

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
LIBDIR = PKG / "_lib"
LIBNAME = "libfa_gpu.so"
CPU_LIBNAME = "libfa_cpu.so"
# measurement only: the read-bandwidth ceiling kernel bench.py reports
READBW_LIBNAME = "libfa_readbw.so"


def library_path() -> Path:
    return LIBDIR / LIBNAME


def cpu_library_path() -> Path:
    return LIBDIR / CPU_LIBNAME


def readbw_library_path() -> Path:
    return LIBDIR / READBW_LIBNAME


def cpu_sources() -> List[Path]:
    return sorted(CSRC.glob("*.cpp"))


def cxx() -> str:
    for cand in (os.environ.get("CXX"), shutil.which("g++"), shutil.which("c++")):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("no host C++ compiler found (set CXX)")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm)")


def archs() -> List[str]:
    env = os.environ.get("FA_HIP_ARCHS", "gfx950")
    return [a for a in env.replace(",", " ").split() if a]


def sources() -> List[Path]:
    return sorted(CSRC.glob("*.hip"))


def headers() -> List[Path]:
    return sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def compile_flags() -> List[str]:
    flags = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", f"-I{INCLUDE}",
             # CDNA4 packed-FP32 forms stay off: plain float code only.
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             # MFMA accumulators in VGPRs: no v_accvgpr_read copies before the VALU uses them
             "-mllvm", "-amdgpu-mfma-vgpr-form",
             # every device atomic here is issued by one lane at an address of
             # its own: the wave-aggregating atomic optimizer only wraps each in a
             # readfirstlane and a wait, serialising the finishes' returning atomics
             "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]
    for a in archs():
        flags.append(f"--offload-arch={a}")
    return flags


def _run(cmd: Sequence[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(list(cmd), stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        # the host pass warns about the gfx-only feature flag; drop that noise
        out = "\n".join(l for l in res.stdout.splitlines()
                        if "is not a recognized feature" not in l)
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")


def build_cpu(verbose: bool = False) -> Path:
    """Compile the host kernels into ``libfa_cpu.so``; returns its path.

    The hot loops are built for AVX2 + FMA; ``fa_cpu_has_avx2`` (compiled into
    the same library, safe on any x86-64) tells the loader whether it may call
    them on the machine at hand.
    """
    LIBDIR.mkdir(exist_ok=True)
    out = cpu_library_path()
    tmp = out.with_name(f".{out.name}.{os.getpid()}.tmp")
    cmd = [cxx(), "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-mavx2", "-mfma",
           "-fvisibility=hidden", "-fno-math-errno", f"-I{INCLUDE}",
           *map(str, cpu_sources()), "-o", str(tmp)]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile every kernel source and link ``libfa_gpu.so`` (and build
    ``libfa_cpu.so``); returns the GPU library's path."""
    build_cpu(verbose)
    cc = hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    flags = compile_flags()
    objs = []
    cmds = []
    for src in sources():
        obj = objdir / (src.stem + ".o")
        objs.append(obj)
        cmds.append([cc, *flags, "-c", str(src), "-o", str(obj)])
    # bench.py's read-bandwidth ceiling kernel, a library of its own
    rb = readbw_library_path()
    rb_tmp = rb.with_name(f".{rb.name}.{os.getpid()}.tmp")
    cmds.append([cc, *flags, "-shared", *map(str, sorted((CSRC / "bench").glob("*.hip"))),
                 "-o", str(rb_tmp)])
    n = jobs or min(len(cmds), max(1, os.cpu_count() or 1))
    with _cf.ThreadPoolExecutor(max_workers=n) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    out = library_path()
    tmp = out.with_name(f".{out.name}.{os.getpid()}.tmp")
    link = [cc, *[f"--offload-arch={a}" for a in archs()], "-shared", "-fPIC",
            *map(str, objs), "-o", str(tmp)]
    _run(link, verbose)
    os.replace(tmp, out)  # atomic: a concurrent loader never sees half a file
    os.replace(rb_tmp, rb)
    return out


def is_stale() -> bool:
    """True when a library is missing or older than any source or header."""
    for lib, srcs in ((library_path(), sources()), (cpu_library_path(), cpu_sources())):
        if not lib.exists():
            return True
        t = lib.stat().st_mtime
        if any(p.stat().st_mtime > t for p in (*srcs, *headers())):
            return True
    return False


if __name__ == "__main__":
    print(build(verbose=True))
