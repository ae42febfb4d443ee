"""Benchmark of the fused metric path on one MI355X; prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Headline (``value``): SSIM forward throughput on configs[1] of BASELINE.json,
an 8x3x1080x1920 uint8 pair (a ~ U{0..255}, b = clip(a + round(N(0, 8)))),
counted as N*C*H*W samples of one input per second (Gpixel/s).  A "step" is
one ``fa.ssim(a, b, data_range=255)`` call (fused kernel + finalize) over one
batch; K steps are timed between device synchronisations, cycling through 4
distinct resident pairs (398 MB) so the 256 MB Infinity Cache cannot serve the
inputs.

Also reported: PSNR on configs[2] (8x3x2160x3840 uint8), as achieved GB/s at 2
bytes per sample and its fraction of the 8 TB/s HBM peak.

``roofline`` is measured live for the dominant kernel (the matrix-core SSIM
kernel, which an fa.ssim call runs as its only launch: it also finishes the
mean): its launches through the C ABI (fa_gpu_ssim_once) are bracketed with
HIP events on the stream they run on, so the average is that kernel alone.  The algorithmic bytes are 2 B per input sample; the kernel
is bound by instruction issue (vector ALU and matrix cores together), so its
arithmetic -- the two 11-tap passes over four moments and the SSIM formula,
counted as float32 operations per output pixel -- is reported beside the HBM
figure.  ``traffic`` is filled from the committed rocprofv3 PMC summary when
present.

Besides: ``latency_single_frame`` (per-call ms at 512^2 and one 1080p frame,
beside the reference's RTX 3090 row), ``streaming`` (``StreamingMetrics``
frames per second at 1080p RGB, host-in and resident) and ``peak_memory_MiB``
(device memory a call allocates above its inputs, forward and loss step at
1080p x8) -- the reference's own measurements of this path.  The MS-SSIM loss
step is timed and measured twice: as shipped (the training forward keeps the
backward's coefficient maps) and with FA_MS_SSIM_RECOMPUTE=1 (recomputed in the
backward, the reference's memory profile).

``cpu_baseline`` times the reference's own CPU kernels (oracle/_ref, compiled
from the reference sources) on a bounded sample of the same workload, on all
host cores.  ``cpu_configs0`` runs configs[0] (1x3x512x512 uint8) through the
``fa.*`` API on CPU tensors -- this build's host library, libfa_cpu.so -- with
the reference CPU build's time for the same kernel beside it.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
BASELINE_GPIXS = 25.6     # reference SSIM Gpixel/s, RTX 3090 (README.md:61)
SSIM_SHAPE = (8, 3, 1080, 1920)
PSNR_SHAPE = (8, 3, 2160, 3840)
# FP32 operations per SSIM output pixel of this kernel at K=11 (fused multiply-
# adds counted as 2): vertical 4 planes x 11 taps, horizontal 4 x 11, moments
# 4 (x', y', x'y', (x'-y')^2 from 2 loads), epilogue 18.
SSIM_FLOP_PER_PIXEL = 2 * 44 + 2 * 44 + 8 + 18
PROFILE_PMC = REPO / "profiles" / "ssim_fwd_1080p8_pmc.txt"
F16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak (no sparsity)
MFMA_FLOP = 16 * 16 * 32 * 2    # one v_mfma_f32_16x16x32_f16


def _pairs(torch, shape, sigma, count, dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    out = []
    for _ in range(count):
        a = torch.randint(0, 256, shape, dtype=torch.uint8, device=dev, generator=g)
        n = torch.round(torch.randn(shape, device=dev, generator=g) * sigma)
        b = (a.to(torch.int16) + n.to(torch.int16)).clamp(0, 255).to(torch.uint8)
        del n
        out.append((a, b))
    return out


def _time_steps(torch, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


LEG_WARMUP_S = 0.2  # untimed calls before each secondary leg
LEG_BATCHES = 5     # a secondary leg reports its fastest batch


def _leg_ms(torch, fn, reps, warmup):
    """Milliseconds per call of a secondary leg: the fastest of LEG_BATCHES
    batches of ``reps`` calls, each batch between synchronisations (the
    reference's timer, bench/bench.py:41-65), so one stall of the box does not
    move a 20-call mean."""
    best = None
    for _ in range(LEG_BATCHES):
        t = _time_steps(torch, fn, reps, warmup) / reps * 1e3
        best = t if best is None else min(best, t)
        warmup = 0
    return best


def _clock_warmup(torch, fn, seconds):
    """Run ``fn`` back to back for ``seconds`` of wall time (untimed).  The
    MI355X raises its clock over ~40 ms (~400 launches of the SSIM kernel) of
    sustained load and drops it again after ~1 s idle: cold, the SSIM kernel
    takes 105-112 us, warm 87-88 us (measured launch by launch).  A short
    warm-up count alone would time the ramp, not the kernel."""
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(50):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    return i


def _kernel_ms(torch, launch, iters):
    """Average duration of `launch` (one kernel) from HIP events on the
    current stream, which is the stream the C ABI launches on."""
    st = torch.cuda.current_stream()
    launch(0)
    st.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(iters):
        launch(i)
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def _pmc_value(key):
    """A figure of the SSIM kernel from the committed PMC summary (its
    ``key: value`` lines), or None."""
    if not PROFILE_PMC.exists():
        return None
    for line in PROFILE_PMC.read_text().splitlines():
        if line.startswith(key + ":"):
            return float(line.split(":", 1)[1])
    return None


def read_ceiling(torch, pairs, block_sizes=(256, 512, 1024), per_cu=(1, 2, 4),
                 unrolls=(2, 4, 8)):
    """The fastest pure read of the same bytes as one PSNR call (both tensors of
    a configs[2] pair, walked in lockstep), over a sweep of launch shapes of
    the read-only kernel in ``csrc/bench/fa_readbw.hip``; the two resident
    pairs rotate so the Infinity Cache cannot serve them.  Returns
    ``(GB/s, shape)``, or None without the kernel library."""
    from frame_analytics_amd import _build

    path = _build.readbw_library_path()
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    fn = lib.fa_readbw_launch
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    sink = torch.zeros(1, dtype=torch.int32, device=pairs[0][0].device)
    nbytes = pairs[0][0].numel()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream

    def run(u, blocks, bs):
        def launch(i):
            a, b = pairs[i % len(pairs)]
            rc = fn(a.data_ptr(), b.data_ptr(), nbytes, u, blocks, bs, sink.data_ptr(), stream)
            assert rc == 0, rc
        return launch

    best = None
    for bs in block_sizes:
        for k in per_cu:
            for u in unrolls:
                ms = _kernel_ms(torch, run(u, cus * k, bs), 20)
                if best is None or ms < best[0]:
                    best = (ms, u, k, bs)
    ms = _kernel_ms(torch, run(best[1], cus * best[2], best[3]), 200)
    shape = {"unroll": best[1], "blocks_per_cu": best[2], "block": best[3]}
    return 2.0 * nbytes / (ms * 1e-3) / 1e9, shape


def cpu_baseline(seconds=12.0):
    """Reference CPU SSIM (oracle/_ref) on 1x3x1080x1920 uint8 pairs, all cores."""
    import numpy as np

    from oracle import ref_cpu

    if not ref_cpu.available():
        return None
    cores = os.cpu_count() or 1
    ref_cpu.load(threads=cores)
    rng = np.random.default_rng(0)
    shape = (1,) + SSIM_SHAPE[1:]
    a = rng.integers(0, 256, shape, dtype=np.uint8)
    b = np.clip(a.astype(np.int16) + np.round(rng.normal(0, 8, shape)).astype(np.int16),
                0, 255).astype(np.uint8)
    ref_cpu.ssim_per_image(a, b)  # warm the pool
    best = float("inf")
    t_end = time.perf_counter() + seconds
    reps = 0
    while reps < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        ref_cpu.ssim_per_image(a, b)
        best = min(best, time.perf_counter() - t0)
        reps += 1
    samples = a.size
    return {"value": round(samples / best / 1e9, 4), "unit": "Gpixel/s", "cores": cores,
            "kind": "reference",
            "sample": f"reference fa_cpu_ssim (oracle/_ref, -O3 -mavx2 -mfma -ffast-math) on "
                      f"1x3x1080x1920 uint8, best of {reps} calls over ~{seconds:.0f} s"}


def _best_of(fn, seconds):
    fn()
    best, reps = float("inf"), 0
    t_end = time.perf_counter() + seconds
    while reps < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        reps += 1
    return best


def _host_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_configs0(seconds=0.6):
    """configs[0] (1x3x512x512 uint8, sigma 8) through fa.* on CPU tensors
    (libfa_cpu.so), each call timed best-of over ~`seconds`; beside it this
    build's host kernel alone (``kernel_ms``) and the reference CPU build's
    kernel for the same call (``reference_kernel_ms``), both through the C ABI."""
    import numpy as np
    import torch

    import frame_analytics_amd as fa
    from frame_analytics_amd import backend
    from oracle import ref_cpu

    if backend.load_cpu() is None:
        return None
    rng = np.random.default_rng(0)
    shape = (1, 3, 512, 512)
    a = rng.integers(0, 256, shape, dtype=np.uint8)
    b = np.clip(a.astype(np.int16) + np.round(rng.normal(0, 8, shape)).astype(np.int16),
                0, 255).astype(np.uint8)
    ta, tb = torch.from_numpy(a), torch.from_numpy(b)
    # this build's host kernels through the same C ABI and arguments as the
    # reference's (oracle/ref_cpu.py), so the two kernel columns compare alike
    mine = backend.load_cpu()
    pa, pb = a.ctypes.data, b.ctypes.data
    n, c, h, w = shape
    win = ref_cpu._window(11, 1.5)

    def my_pixel(bias):
        out = np.zeros(1, np.float64)
        assert mine.fa_cpu_pixel_reduce(pa, pb, 0, n, a.size // n, 0, 0.0, bias, 0,
                                        out.ctypes.data) == 0

    def my_ssim():
        per_plane = np.zeros(n * c, np.float64)
        assert mine.fa_cpu_ssim(pa, pb, 0, n, c, h, w, win.ctypes.data, 11, 127.5,
                                (0.01 * 255) ** 2, (0.03 * 255) ** 2, None,
                                per_plane.ctypes.data) == 0

    def my_gmsd():
        mean, std = np.zeros(n, np.float64), np.zeros(n, np.float64)
        assert mine.fa_cpu_gmsd(pa, pb, 0, n, c, h, w, 170.0, (1e-6 * 255) ** 2, 1,
                                mean.ctypes.data, std.ctypes.data) == 0

    bias = 20 * np.log10(255.0)
    calls = {
        "ssim": (lambda: fa.ssim(ta, tb, data_range=255.0), my_ssim,
                 lambda: ref_cpu.ssim_per_image(a, b)),
        "psnr": (lambda: fa.psnr(ta, tb), lambda: my_pixel(bias),
                 lambda: ref_cpu.pixel_reduce(a, b, "mse", psnr_bias=bias)),
        "mse": (lambda: fa.mse(ta, tb), lambda: my_pixel(-1e300),
                lambda: ref_cpu.pixel_reduce(a, b, "mse")),
        "gmsd": (lambda: fa.gmsd(ta, tb, data_range=255.0), my_gmsd,
                 lambda: ref_cpu.gmsd(a, b)),
        "ms_ssim": (lambda: fa.ms_ssim(ta, tb, data_range=255.0), None, None),
    }
    have_ref = ref_cpu.available()
    if have_ref:
        ref_cpu.load(threads=torch.get_num_threads())
    out = {"workload": "1x3x512x512 uint8 (configs[0]), fa.* on CPU tensors",
           "host": f"{_host_model()}, {os.cpu_count()} logical CPUs, "
                   f"{torch.get_num_threads()} threads"}
    for name, (call, kern, theirs) in calls.items():
        row = {"ms": round(_best_of(call, seconds) * 1e3, 4)}
        if kern is not None:
            row["kernel_ms"] = round(_best_of(kern, seconds) * 1e3, 4)
        if theirs is not None and have_ref:
            row["reference_kernel_ms"] = round(_best_of(theirs, seconds) * 1e3, 4)
        out[name] = row
    return out


def profile_sequence(launches=20):
    """A fixed launch sequence for rocprofv3 counter runs (``--profile``):
    a torch copy of exactly 256 MiB (the FETCH_SIZE / WRITE_SIZE calibration:
    256 MiB read, 256 MiB written), then `launches` launches each of the SSIM
    kernel (configs[1]; the one-launch mean, then with the float32 map), the
    GMSD kernel (configs[4], one launch), MS-SSIM (configs[4], three launches)
    and the PSNR pixel kernel (configs[2], one launch), through the C ABI,
    rotating resident input pairs."""
    import torch

    import frame_analytics_amd as fa
    from frame_analytics_amd import backend

    dev = torch.device("cuda:0")
    ext = backend.load()
    lib = ext.gpu
    stream = torch.cuda.current_stream().cuda_stream
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

    pairs = _pairs(torch, SSIM_SHAPE, 8.0, 4, dev, seed=1)
    n, c, h, w = SSIM_SHAPE
    win = fa.gaussian_window_1d(11, 1.5, device=dev, dtype=torch.float32)
    bpp = backend.workspace_slots("ssim", h, w, 11)
    partial = torch.empty((n * c, bpp), dtype=torch.float64, device=dev)
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=dev)
    tot = torch.empty((), dtype=torch.float64, device=dev)
    for i in range(launches):
        a, b = pairs[i % 4]
        assert lib.fa_gpu_ssim_once(a.data_ptr(), b.data_ptr(), 0, n, c, h, w, None, None, None,
                                    win.data_ptr(), 11, 127.5, (0.01 * 255) ** 2,
                                    (0.03 * 255) ** 2, None, partial.data_ptr(), bpp,
                                    acc.data_ptr(), None, tot.data_ptr(), 0, stream) == 0
    torch.cuda.synchronize()
    # the same kernel writing the float32 map (configs[1], return_map=True)
    smap = torch.empty((n, c, h - 10, w - 10), dtype=torch.float32, device=dev)
    for i in range(launches):
        a, b = pairs[i % 4]
        assert lib.fa_gpu_ssim(a.data_ptr(), b.data_ptr(), 0, n, c, h, w, win.data_ptr(), 11,
                               127.5, (0.01 * 255) ** 2, (0.03 * 255) ** 2, smap.data_ptr(),
                               partial.data_ptr(), bpp, None, None, 0, stream) == 0
    torch.cuda.synchronize()
    del smap
    # GMSD (configs[4]: downsample, per-channel pooled) on the same pairs
    gbpp = backend.workspace_slots("gmsd", h, w, 1)
    ps = torch.empty((n * c, gbpp), dtype=torch.float64, device=dev)
    ps2 = torch.empty_like(ps)
    gm = torch.empty(n, dtype=torch.float64, device=dev)
    gs = torch.empty_like(gm)
    gacc = torch.zeros(backend._ACC_WORDS["gmsd"], dtype=torch.int64, device=dev)
    for i in range(launches):
        a, b = pairs[i % 4]
        assert lib.fa_gpu_gmsd_once(a.data_ptr(), b.data_ptr(), 0, n, c, h, w, None, None, None,
                                    170.0, (255e-6) ** 2, 1, ps.data_ptr(), ps2.data_ptr(), gbpp,
                                    gacc.data_ptr(), gm.data_ptr(), gs.data_ptr(), None, 0,
                                    stream) == 0
    torch.cuda.synchronize()
    # MS-SSIM (configs[4], 5 scales: the three-launch form with the stream's
    # accumulator, fa.ms_ssim's inference call) on the same pairs
    from frame_analytics_amd.functional import MS_SSIM_WEIGHTS

    mbytes = backend._ms_workspace_bytes(0, n, c, h, w, 11, 5, False)
    mws = torch.empty(mbytes, dtype=torch.uint8, device=dev)
    macc = torch.zeros(backend._ACC_WORDS["ms"], dtype=torch.int64, device=dev)
    wts = (ctypes.c_double * 5)(*MS_SSIM_WEIGHTS)
    for i in range(launches):
        a, b = pairs[i % 4]
        assert lib.fa_gpu_ms_ssim(a.data_ptr(), b.data_ptr(), 0, n, c, h, w, None, None, None,
                                  win.data_ptr(), 11, 127.5, (0.01 * 255) ** 2,
                                  (0.03 * 255) ** 2, wts, 5, mws.data_ptr(), mbytes,
                                  macc.data_ptr(), None, tot.data_ptr(), 0, stream) == 0
    torch.cuda.synchronize()
    del pairs, partial, ps, ps2, mws

    ppairs = _pairs(torch, PSNR_SHAPE, 4.0, 2, dev, seed=2)
    pn = PSNR_SHAPE[0]
    per = ppairs[0][0].numel() // pn
    bpi = backend.workspace_slots("pixel", pn, per, 0)
    ppart = torch.empty((pn, bpi), dtype=torch.float64, device=dev)
    pacc = torch.zeros(backend._ACC_WORDS["pixel"], dtype=torch.int64, device=dev)
    pdb = torch.empty((), dtype=torch.float64, device=dev)
    for i in range(launches):
        a, b = ppairs[i % 2]
        assert lib.fa_gpu_pixel_reduce_once(a.data_ptr(), b.data_ptr(), 0, pn, per, 0, 0.0,
                                            10.0 * math.log10(255.0 ** 2), ppart.data_ptr(), bpi,
                                            pacc.data_ptr(), None, None, None, pdb.data_ptr(), 0,
                                            stream) == 0
    torch.cuda.synchronize()
    print("profile sequence done", flush=True)


def trace_leg(name, steps, warmup):
    """One training leg alone, for a kernel trace of its forward and backward
    kernels (``--trace-leg``): ``configs3`` is 1 - ssim(x, y) on
    16x3x256x256 float32, ``msssim_loss`` 1 - ms_ssim(x, y) on the configs[4]
    frames as float32 in [0, 1].  Prints the step time."""
    import torch

    import frame_analytics_amd as fa

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    if name == "configs3":
        x = torch.rand((16, 3, 256, 256), device=dev, generator=g)
        y = (x + 0.05 * torch.randn(x.shape, device=dev, generator=g)).clamp(0, 1)
        fn = fa.ssim
    elif name == "msssim_loss":
        a, b = _pairs(torch, SSIM_SHAPE, 8.0, 1, dev, seed=1)[0]
        x, y = a.float() / 255.0, b.float() / 255.0
        fn = fa.ms_ssim
    else:
        raise SystemExit(f"unknown leg {name!r}")
    x.requires_grad_(True)

    def step(i):
        x.grad = None
        (1.0 - fn(x, y, data_range=1.0)).backward()

    _clock_warmup(torch, step, 0.3)
    ms = _time_steps(torch, step, steps, warmup) / steps * 1e3
    print(json.dumps({"leg": name, "steps": steps, "ms_per_step": round(ms, 4)}), flush=True)


def _frames(torch, shape, dev, seed, sigma=8.0):
    """One resident uint8 pair of ``shape`` (the BASELINE.json generator)."""
    return _pairs(torch, shape, sigma, 1, dev, seed)[0]


# The reference's per-call table (README.md:53-59, RTX 3090), ms: SSIM and
# PSNR on one channel (its bench/bench.py:188), MS-SSIM / GMSD / L1 on three
# (bench/bench_training.py:127,232,269).
REF_LATENCY_MS = {
    "ssim": {"512": 0.024, "1080p": 0.085}, "psnr": {"512": 0.020, "1080p": 0.028},
    "ms_ssim": {"512": 0.331, "1080p": 0.512}, "gmsd": {"512": 0.023, "1080p": 0.055},
    "l1": {"512": 0.021, "1080p": 0.026},
}


def latency_legs(torch, fa, dev):
    """Per-call milliseconds of single frames, the reference's timer (fastest
    of 5 batches of 20 calls between synchronisations), beside its RTX 3090
    row.  Small frames are where fixed costs show: launches and the Python
    path."""
    out = {"workload": "one frame per call: ssim / psnr 1 channel, ms_ssim / gmsd / l1 "
                       "3 channels (the reference's bench channel counts), uint8"}
    calls = {"ssim": lambda a, b: fa.ssim(a, b, data_range=255.0),
             "psnr": lambda a, b: fa.psnr(a, b, data_range=255.0),
             "ms_ssim": lambda a, b: fa.ms_ssim(a, b, data_range=255.0),
             "gmsd": lambda a, b: fa.gmsd(a, b, data_range=255.0),
             "l1": lambda a, b: fa.l1(a, b)}
    for size, (h, w) in (("512", (512, 512)), ("1080p", (1080, 1920))):
        pairs = {c: _frames(torch, (1, c, h, w), dev, seed=40 + c) for c in (1, 3)}
        for name, fn in calls.items():
            a, b = pairs[1 if name in ("ssim", "psnr") else 3]
            f = (lambda i, fn=fn, a=a, b=b: fn(a, b))
            _clock_warmup(torch, f, 0.1)
            out.setdefault(name, {})[size] = round(_leg_ms(torch, f, 20, 5), 4)
    out["reference_rtx3090_ms"] = REF_LATENCY_MS
    return out


def streaming_leg(torch, fa, dev, frames=300):
    """``StreamingMetrics`` at 1080p RGB (mse + psnr + ssim as one captured HIP
    graph): host uint8 frames in, Python floats out, and the reference's
    resident comparison (fa.ssim + fa.psnr on resident frames), as its
    bench/bench.py:302-335 times them."""
    h, w = 1080, 1920
    g = torch.Generator()
    g.manual_seed(5)
    host = []
    for _ in range(4):
        a = torch.randint(0, 256, (3, h, w), dtype=torch.uint8, generator=g)
        n = torch.round(torch.randn((3, h, w), generator=g) * 8.0).to(torch.int16)
        host.append((a, (a.to(torch.int16) + n).clamp(0, 255).to(torch.uint8)))
    sm = fa.StreamingMetrics((1, 3, h, w), device=dev, dtype=torch.uint8, data_range=255.0)
    for i in range(16):
        sm.update(*host[i % 4])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(frames):
        sm.update(*host[i % 4])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ra, rb = host[0][0].to(dev)[None], host[0][1].to(dev)[None]
    for _ in range(16):
        fa.ssim(ra, rb, data_range=255.0)
        fa.psnr(ra, rb, data_range=255.0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(frames):
        fa.ssim(ra, rb, data_range=255.0)
        fa.psnr(ra, rb, data_range=255.0)
    torch.cuda.synchronize()
    dt2 = time.perf_counter() - t0
    return {"workload": f"{frames} frames of 1080p RGB uint8",
            "graph_captured": bool(sm.graph_captured),
            "host_in_fps": round(frames / dt, 1),
            "resident_fps": round(frames / dt2, 1),
            "reference_rtx3090_fps": {"host_in": 931, "resident": 2941}}


def memory_legs(torch, fa, dev):
    """Peak device allocation of one call above its inputs, MiB (the
    reference's cuda_peak, bench/bench_memory.py:56-86: warm first, then
    max_memory_allocated over the call against what was allocated before),
    at 1080p x8 RGB, beside its RTX 3090 figures (README.md:95-115,150-165)."""
    import gc

    mib = float(1 << 20)

    def peak(fn, setup=None):
        fn()
        if setup is not None:
            setup()
        torch.cuda.synchronize()
        gc.collect()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        before = torch.cuda.memory_allocated()
        out = fn()
        torch.cuda.synchronize()
        v = (torch.cuda.max_memory_allocated() - before) / mib
        del out
        return round(v, 3)

    x8, y8 = _frames(torch, SSIM_SHAPE, dev, seed=9)
    res = {"workload": "8x3x1080x1920: forward on uint8, loss step (forward + backward) "
                       "on float32 frames / 255"}
    with torch.no_grad():
        res["forward"] = {
            "ssim": peak(lambda: fa.ssim(x8, y8, data_range=255.0)),
            "ms_ssim": peak(lambda: fa.ms_ssim(x8, y8, data_range=255.0)),
            "gmsd": peak(lambda: fa.gmsd(x8, y8, data_range=255.0)),
            "psnr": peak(lambda: fa.psnr(x8, y8, data_range=255.0)),
        }
    x = (x8.float() / 255.0).requires_grad_(True)
    y = y8.float() / 255.0
    del x8, y8

    def step(fn):
        def run():
            loss = fn()
            loss.backward()
            return loss
        return run

    def drop_grad():
        x.grad = None

    res["loss_step"] = {
        "ssim": peak(step(lambda: 1.0 - fa.ssim(x, y, data_range=1.0)), drop_grad),
        "ms_ssim": peak(step(lambda: 1.0 - fa.ms_ssim(x, y, data_range=1.0)), drop_grad),
    }
    # with the coefficient maps recomputed in the backward (FA_MS_SSIM_RECOMPUTE=1)
    os.environ["FA_MS_SSIM_RECOMPUTE"] = "1"
    try:
        res["loss_step"]["ms_ssim_recompute"] = peak(
            step(lambda: 1.0 - fa.ms_ssim(x, y, data_range=1.0)), drop_grad)
    finally:
        os.environ.pop("FA_MS_SSIM_RECOMPUTE", None)
    res["reference_rtx3090_MiB"] = {"forward": {"ssim": 0.19, "ms_ssim": 120, "gmsd": 0.19,
                                                "psnr": 0.007},
                                    "loss_step": {"ssim": 752, "ms_ssim": 942}}
    del x, y
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--clock-warmup", type=float, default=0.5,
                    help="seconds of untimed SSIM steps before the warm-up steps "
                         "(the part raises its clock over ~40 ms of load)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile", action="store_true",
                    help="run the fixed launch sequence for rocprofv3 counters and exit")
    ap.add_argument("--trace-leg", choices=("configs3", "msssim_loss"),
                    help="run one training leg alone (for a kernel trace) and exit")
    args = ap.parse_args()
    if args.profile:
        profile_sequence()
        return
    if args.trace_leg:
        trace_leg(args.trace_leg, args.steps, args.warmup)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the per-shard kernel is the single-GPU one; each GPU would run it on its own "
              "images and exchange per-image sums once).", file=sys.stderr)
        sys.exit(2)

    import torch

    import frame_analytics_amd as fa
    from frame_analytics_amd import backend

    dev = torch.device("cuda:0")
    ext = backend.load()
    assert ext is not None and ext.has_gpu, "gfx950 kernel library did not load"
    lib = ext.gpu

    # ---------------- SSIM, configs[1] ---------------------------------- #
    pairs = _pairs(torch, SSIM_SHAPE, 8.0, 4, dev, seed=1)
    n, c, h, w = SSIM_SHAPE
    samples = n * c * h * w

    def ssim_step(i):
        a, b = pairs[i % len(pairs)]
        return fa.ssim(a, b, data_range=255.0)

    warm_calls = _clock_warmup(torch, ssim_step, args.clock_warmup)
    elapsed = _time_steps(torch, ssim_step, args.steps, args.warmup)
    ms_per_step = elapsed / args.steps * 1e3
    gpix = samples * args.steps / elapsed / 1e9

    # dominant kernel alone: the C ABI with no finalize sinks launches only it
    win = fa.gaussian_window_1d(11, 1.5, device=dev, dtype=torch.float32)
    bpp = backend.workspace_slots("ssim", h, w, 11)
    partial = torch.empty((n * c, bpp), dtype=torch.float64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    # the kernel an fa.ssim call runs, alone: fa_gpu_ssim_once finishes the
    # batch mean inside its one launch
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=dev)
    ktot = torch.empty((), dtype=torch.float64, device=dev)

    def ssim_kernel(i):
        a, b = pairs[i % len(pairs)]
        rc = lib.fa_gpu_ssim_once(a.data_ptr(), b.data_ptr(), 0, n, c, h, w, None, None, None,
                                  win.data_ptr(), 11, 127.5, (0.01 * 255) ** 2,
                                  (0.03 * 255) ** 2, None, partial.data_ptr(), bpp,
                                  acc.data_ptr(), None, ktot.data_ptr(), 0, stream)
        assert rc == 0, rc

    k_ms = _kernel_ms(torch, ssim_kernel, 200)
    bytes_per_launch = 2.0 * samples
    achieved = bytes_per_launch / (k_ms * 1e-3) / 1e9
    out_px = n * c * (h - 10) * (w - 10)
    tflops = out_px * SSIM_FLOP_PER_PIXEL / (k_ms * 1e-3) / 1e12
    mfma_count = _pmc_value("mfma_instructions_per_launch")
    mfma_tf = (None if mfma_count is None
               else round(mfma_count * MFMA_FLOP / (k_ms * 1e-3) / 1e12, 2))

    reps = max(20, args.steps // 10)
    # ---------------- MS-SSIM and GMSD on the same pairs ---- #
    c4 = {"workload": "8x3x1080x1920 uint8 (configs[4]), 4 resident pairs rotated"}
    for key, fn in (
            ("ms_ssim_ms", lambda i: fa.ms_ssim(*pairs[i % 4], data_range=255.0)),
            ("gmsd_ms", lambda i: fa.gmsd(*pairs[i % 4], data_range=255.0)),
            ("gmsd_luma_bt601_ms",
             lambda i: fa.gmsd(*pairs[i % 4], data_range=255.0, luma="bt601"))):
        # each leg raises the clock itself: between the legs it may drop
        _clock_warmup(torch, fn, LEG_WARMUP_S)
        c4[key] = round(_leg_ms(torch, fn, reps, 5), 4)
    c4["gmsd_GBps"] = round(2.0 * samples / (c4["gmsd_ms"] * 1e-3) / 1e9, 1)
    l1_fn = lambda i: fa.l1(*pairs[i % 4])  # noqa: E731
    _clock_warmup(torch, l1_fn, LEG_WARMUP_S)
    c4["l1_ms"] = round(_leg_ms(torch, l1_fn, reps, 5), 4)
    del partial
    # MS-SSIM as a training loss (the reference's bench_training.py:172-200 step):
    # x = frames / 255 in float32 with requires_grad, loss = 1 - ms_ssim, backward
    xl = (pairs[0][0].float() / 255.0).requires_grad_(True)
    yl = pairs[0][1].float() / 255.0
    del pairs
    torch.cuda.empty_cache()

    def msssim_loss_step(i):
        xl.grad = None
        (1.0 - fa.ms_ssim(xl, yl, data_range=1.0)).backward()

    lreps = max(5, reps // 4)
    _clock_warmup(torch, msssim_loss_step, LEG_WARMUP_S)
    c4["ms_ssim_loss_fwd_bwd_fp32_ms"] = round(
        _leg_ms(torch, msssim_loss_step, lreps, 2), 3)
    # the same step with the coefficient maps recomputed in the backward (the
    # reference's memory profile, FA_MS_SSIM_RECOMPUTE=1)
    os.environ["FA_MS_SSIM_RECOMPUTE"] = "1"
    try:
        c4["ms_ssim_loss_fwd_bwd_fp32_recompute_ms"] = round(
            _leg_ms(torch, msssim_loss_step, lreps, 2), 3)
    finally:
        os.environ.pop("FA_MS_SSIM_RECOMPUTE", None)
    del xl, yl
    # the reference's published RTX 3090 figures for the same calls (its README)
    c4["reference_rtx3090_ms"] = {"ms_ssim": 3.088, "gmsd": 0.313, "l1": 0.115,
                                  "ms_ssim_loss_fwd_bwd_fp32": 12.7}
    torch.cuda.empty_cache()

    # ---------------- SSIM loss, forward + backward -------- #
    g3 = torch.Generator(device=dev)
    g3.manual_seed(3)
    x3 = torch.rand((16, 3, 256, 256), device=dev, generator=g3)
    y3 = (x3 + 0.05 * torch.randn(x3.shape, device=dev, generator=g3)).clamp(0, 1)
    x3.requires_grad_(True)

    def loss_step(i):
        x3.grad = None
        (1.0 - fa.ssim(x3, y3, data_range=1.0)).backward()

    _clock_warmup(torch, loss_step, LEG_WARMUP_S)
    c3_ms = _leg_ms(torch, loss_step, reps, 5)
    # The same step with the autograd engine running the backward in the
    # calling thread: by default it hands a GPU graph to its device thread and
    # waits, and on these hosts that round trip costs more than the step's
    # kernels (~0.15 ms of host time per step against ~85 us of kernels).
    with torch.autograd.set_multithreading_enabled(False):
        _clock_warmup(torch, loss_step, LEG_WARMUP_S)
        c3_inline_ms = _leg_ms(torch, loss_step, reps, 5)
    del x3, y3

    # ---------------- PSNR, configs[2] ---------------------------------- #
    ppairs = _pairs(torch, PSNR_SHAPE, 4.0, 2, dev, seed=2)
    pn = PSNR_SHAPE[0]
    per = ppairs[0][0].numel() // pn

    def psnr_step(i):
        a, b = ppairs[i % len(ppairs)]
        return fa.psnr(a, b, data_range=255.0)

    _clock_warmup(torch, psnr_step, LEG_WARMUP_S)
    p_ms = _leg_ms(torch, psnr_step, reps, 5)
    pbytes = 2.0 * ppairs[0][0].numel()
    bpi = backend.workspace_slots("pixel", pn, per, 0)
    ppart = torch.empty((pn, bpi), dtype=torch.float64, device=dev)

    # the one launch an fa.psnr call makes (the sweep that also finishes the
    # batch's dB), alone
    pacc = torch.zeros(backend._ACC_WORDS["pixel"], dtype=torch.int64, device=dev)
    pdb = torch.empty((), dtype=torch.float64, device=dev)

    def psnr_kernel(i):
        a, b = ppairs[i % len(ppairs)]
        rc = lib.fa_gpu_pixel_reduce_once(a.data_ptr(), b.data_ptr(), 0, pn, per, 0, 0.0,
                                          10.0 * math.log10(255.0 ** 2), ppart.data_ptr(), bpi,
                                          pacc.data_ptr(), None, None, None, pdb.data_ptr(), 0,
                                          stream)
        assert rc == 0, rc

    pk_ms = _kernel_ms(torch, psnr_kernel, 200)
    ceiling = read_ceiling(torch, ppairs)
    del ppairs, ppart
    torch.cuda.empty_cache()

    # ---------------- configs[1]'s other two outputs -------------------- #
    # per-image values and the float32 map (8x3x1070x1910, 196 MB written per
    # call besides the 99.5 MB read).  Last, on fresh pairs: the map calls
    # leave 196 MB blocks in the caching allocator, and a training leg timed
    # after them read ~9 ms per step instead of ~1.6 in some runs.
    pairs = _pairs(torch, SSIM_SHAPE, 8.0, 4, dev, seed=1)
    c1 = {"workload": "fa.ssim on configs[1], 4 resident pairs rotated"}
    map_bytes = 4.0 * n * c * (h - 10) * (w - 10)
    for key, fn in (
            ("none_ms", lambda i: fa.ssim(*pairs[i % 4], data_range=255.0, reduction="none")),
            ("map_ms", lambda i: fa.ssim(*pairs[i % 4], data_range=255.0, return_map=True))):
        _clock_warmup(torch, fn, LEG_WARMUP_S)
        c1[key] = round(_leg_ms(torch, fn, reps, 5), 4)
    c1["map_GBps"] = round((bytes_per_launch + map_bytes) / (c1["map_ms"] * 1e-3) / 1e9, 1)
    del pairs
    torch.cuda.empty_cache()
    torch.cuda.empty_cache()

    latency = latency_legs(torch, fa, dev)
    streaming = streaming_leg(torch, fa, dev)
    memory = memory_legs(torch, fa, dev)

    line = {
        "metric": "SSIM Gpixel/s at 1080p x8 uint8 (configs[1]); PSNR 4K x8 HBM GB/s beside it",
        "value": round(gpix, 3),
        "unit": "Gpixel/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(gpix / BASELINE_GPIXS, 3),
        # the input samples; the kernel multiplies exact fp16 hi + lo pieces
        # of them on the matrix cores and accumulates in float32
        "dtype": "u8",
        "operands": "fp16 hi+lo split operands (v_mfma_f32_16x16x32_f16), f32 accumulate",
        "data": "synthetic uint8 (BASELINE.json generator, 4 resident pairs rotated); "
                f"{args.clock_warmup:g} s clock warm-up ({warm_calls} untimed steps) before "
                f"the warm-up steps; {LEG_WARMUP_S:g} s of untimed calls before each "
                "secondary leg",
        "config": {"workload": "ssim_fwd 8x3x1080x1920 uint8, reduction=mean, 11x11 gaussian",
                   "batch": n, "channels": c, "height": h, "width": w},
        "roofline": {
            # the north star prices SSIM against HBM; the kernel itself is
            # bound by instruction issue (vector ALU and matrix cores), see
            # "limiter" and the busy fractions below
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _pmc_value("traffic_bytes_per_launch"),
            "kernel": "ssim_mfma_kernel<uint8,REDUCE,finish> (v_mfma_f32_16x16x32_f16 passes)",
            "kernel_ms": round(k_ms, 4),
            "limiter": "instruction issue (VALU + MFMA), not HBM",
            # the filter and formula work as float32 operations per output
            # pixel (202 at K = 11), over the kernel time
            "arith_tflops_f32_equiv": round(tflops, 2),
            # what the matrix cores execute: fp16 hi/lo pieces, f32 accumulate
            "mfma_tflops_f16": mfma_tf,
            "mfma_frac_of_f16_dense_peak": (None if mfma_tf is None
                                            else round(mfma_tf / F16_DENSE_PEAK_TFLOPS, 4)),
            "mfma_busy": _pmc_value("mfma_busy"),
            "valu_busy": _pmc_value("valu_busy"),
        },
        "psnr": {
            "workload": "psnr 8x3x2160x3840 uint8 (configs[2]), 2 resident pairs rotated",
            "ms_per_step": round(p_ms, 4),
            "GBps_end_to_end": round(pbytes / (p_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak_end_to_end": round(pbytes / (p_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": "pix_sweep_kernel<uint8,MSE> finishing the dB in its launch",
            "kernel_ms": round(pk_ms, 4),
            "GBps_kernel": round(pbytes / (pk_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(pbytes / (pk_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "read_ceiling_GBps": None if ceiling is None else round(ceiling[0], 1),
            "read_ceiling_frac_of_hbm_peak": (None if ceiling is None
                                              else round(ceiling[0] / HBM_PEAK_GBS, 4)),
            "read_ceiling_shape": None if ceiling is None else ceiling[1],
            "frac_of_read_ceiling": (None if ceiling is None
                                     else round(pbytes / (pk_ms * 1e-3) / 1e9 / ceiling[0], 4)),
        },
        "configs4": c4,
        "configs3": {"workload": "1 - ssim(x, y) forward + backward, 16x3x256x256 float32",
                     "ms_per_step": round(c3_ms, 4),
                     "ms_per_step_backward_in_calling_thread": round(c3_inline_ms, 4)},
        "configs1_other_outputs": c1,
        "latency_single_frame": latency,
        "streaming": streaming,
        "peak_memory_MiB": memory,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(),
        "cpu_configs0": None if args.no_cpu_baseline else cpu_configs0(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
