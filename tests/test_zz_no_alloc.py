"""fa_gpu_ssim_noalloc: fa_gpu_ssim without a caller workspace.

The no-allocation entry point runs the same kernels as fa_gpu_ssim with the
partial sums in the library's fixed scratch array, so its outputs must equal
fa_gpu_ssim's bit for bit: checked on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents), for the uint8
matrix-core kernel, the float32 strip kernel and the map mode, and against the
oracle at configs[1] size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as ref
from tests.conftest import u8_pair

pytestmark = pytest.mark.gpu

C1, C2 = (0.01 * 255.0) ** 2, (0.03 * 255.0) ** 2
_CODE = {torch.uint8: 0, torch.float32: 3}


def _window(dev):
    import frame_analytics_amd as fa

    return fa.gaussian_window_1d(11, 1.5, device=dev, dtype=torch.float32)


def _outputs(x, with_map):
    n, c, h, w = x.shape
    per = torch.full((n,), -7.0, dtype=torch.float64, device=x.device)
    tot = torch.full((), -7.0, dtype=torch.float64, device=x.device)
    smap = (torch.full((n, c, h - 10, w - 10), -7.0, dtype=torch.float32, device=x.device)
            if with_map else None)
    return per, tot, smap


def _ptr(t):
    return None if t is None else t.data_ptr()


def _with_workspace(x, y, with_map):
    from frame_analytics_amd import backend

    n, c, h, w = (int(v) for v in x.shape)
    bpp = backend.workspace_slots("ssim", h, w, 11)
    partial = torch.empty((n * c, bpp), dtype=torch.float64, device=x.device)
    per, tot, smap = _outputs(x, with_map)
    win = _window(x.device)
    rc = backend.call_gpu("fa_gpu_ssim", x.data_ptr(), y.data_ptr(), _CODE[x.dtype], n, c, h,
                          w, win.data_ptr(), 11, 127.5, C1, C2, _ptr(smap), partial.data_ptr(),
                          bpp, per.data_ptr(), tot.data_ptr(), 0,
                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return per, tot, smap


def _no_alloc(x, y, with_map):
    from frame_analytics_amd import backend

    n, c, h, w = (int(v) for v in x.shape)
    per, tot, smap = _outputs(x, with_map)
    win = _window(x.device)
    rc = backend.call_gpu("fa_gpu_ssim_noalloc", x.data_ptr(), y.data_ptr(), _CODE[x.dtype],
                          n, c, h, w, win.data_ptr(), 11, 127.5, C1, C2, _ptr(smap),
                          per.data_ptr(), tot.data_ptr(), 0,
                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return per, tot, smap


def _same(a, b):
    for u, v in zip(a, b):
        if u is None:
            assert v is None
            continue
        assert torch.equal(u, v), (u.flatten()[:4], v.flatten()[:4])


@pytest.mark.parametrize("dtype", [torch.uint8, torch.float32])
def test_noalloc_equals_workspace_call_twice(gpu, dtype):
    """configs[1] (8x3x1080x1920), then a smaller batch: each call's
    per-image and batch means equal fa_gpu_ssim's, bit for bit."""
    first = u8_pair((8, 3, 1080, 1920), 8.0, seed=1)
    second = u8_pair((2, 1, 300, 416), 12.0, seed=2)
    for k, (a, b) in enumerate((first, second)):
        print(f"noalloc call {k}: shape {a.shape} {dtype}", flush=True)
        x = torch.from_numpy(a).to(gpu).to(dtype)
        y = torch.from_numpy(b).to(gpu).to(dtype)
        want = _with_workspace(x, y, False)
        got = _no_alloc(x, y, False)
        torch.cuda.synchronize()
        _same(got, want)
        if k == 0 and dtype == torch.uint8:
            o = ref.ssim(a[:1], b[:1], 255.0)
            assert abs(float(got[0][0]) - o) <= 1e-6 * o


def test_noalloc_map_mode_twice(gpu):
    """The map and the means, larger call then smaller call."""
    for k, shape in enumerate(((2, 3, 520, 712), (1, 2, 64, 96))):
        a, b = u8_pair(shape, 10.0, seed=10 + k)
        x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
        want = _with_workspace(x, y, True)
        got = _no_alloc(x, y, True)
        torch.cuda.synchronize()
        _same(got, want)
        if k == 1:
            m = ref.ssim(a, b, 255.0, return_map=True)
            assert np.abs(got[2].double().cpu().numpy() - m).max() < 5e-6


def test_noalloc_rejects_oversize_before_the_gpu(gpu):
    from frame_analytics_amd import backend

    slots = backend.workspace_slots("ssim", 2160, 3840, 11)
    too_many = (1 << 20) // slots + 1
    rc = backend.call_gpu("fa_gpu_ssim_noalloc", None, None, 0, too_many, 1, 2160, 3840, None,
                          11, 127.5, C1, C2, None, None, None, 0, None)
    assert rc == 8  # FA_E_SCRATCH
    assert b"scratch" in backend.load().gpu.fa_gpu_error_string(8)


def test_noalloc_captured_in_a_graph_and_replayed(gpu):
    """After one eager call on the device, fa_gpu_ssim_noalloc is captured
    into a HIP graph (torch.cuda.CUDAGraph) over static input and output
    buffers; each replay on new frames -- with eager calls of the library
    between replays -- gives fa_gpu_ssim's eager means bit for bit."""
    from frame_analytics_amd import backend

    shape = (2, 3, 256, 384)
    a0, b0 = u8_pair(shape, 9.0, seed=20)
    x = torch.from_numpy(a0).to(gpu)
    y = torch.from_numpy(b0).to(gpu)
    n, c, h, w = shape
    per, tot, _ = _outputs(x, False)
    win = _window(gpu)

    def call(stream):
        return backend.call_gpu("fa_gpu_ssim_noalloc", x.data_ptr(), y.data_ptr(), 0, n, c, h,
                                w, win.data_ptr(), 11, 127.5, C1, C2, None, per.data_ptr(),
                                tot.data_ptr(), 0, stream)

    assert call(torch.cuda.current_stream().cuda_stream) == 0  # the eager first call
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert call(torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    for k in range(3):
        a, b = u8_pair(shape, 6.0 + 3 * k, seed=21 + k)
        print(f"graph replay {k}", flush=True)
        x.copy_(torch.from_numpy(a))
        y.copy_(torch.from_numpy(b))
        graph.replay()
        got = (per.clone(), tot.clone())
        torch.cuda.synchronize()
        want = _with_workspace(x, y, False)  # eager, between the replays
        torch.cuda.synchronize()
        _same(got, want[:2])
        o = ref.ssim(a[:1], b[:1], 255.0)
        assert abs(float(got[0][0]) - o) <= 1e-6 * o
