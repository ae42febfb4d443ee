"""GPU parity of the pixel reductions (MSE / PSNR / L1 / Charbonnier / Huber).

Bar: uint8 MSE and L1 are bit-exact against integer sums (the oracle's int64
SSE/SAD divided once by the count); PSNR matches 10 log10(L^2) - 10 log10(mse)
to 1e-12 (device and host log10 may differ in the last ulp); float ops are
within 1e-9 relative of float64 (Charbonnier on non-float64 input: 1e-6, its
square root is float32 like the reference's).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import u8_pair

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("shape", [(1, 1, 33, 41), (2, 3, 64, 64), (5, 1, 97, 131),
                                   (3, 3, 127, 233), (1, 3, 512, 512), (4, 2, 1, 4099)])
def test_mse_psnr_l1_u8_bit_exact(gpu, shape):
    a, b = u8_pair(shape, 8.0, seed=sum(shape))
    ta, tb = _t(a, gpu), _t(b, gpu)
    for red in ("mean", "none"):
        got = fa.mse(ta, tb, reduction=red).cpu().numpy()
        want = ref.mse(a, b, red)
        assert np.array_equal(got, np.asarray(want)), (red, got, want)
        got_l1 = fa.l1(ta, tb, reduction=red).cpu().numpy()
        assert np.array_equal(got_l1, np.asarray(ref.l1(a, b, red)))
        p = fa.psnr(ta, tb, data_range=255.0, reduction=red).cpu().numpy()
        assert np.allclose(p, ref.psnr(a, b, 255.0, red), rtol=1e-12, atol=0)


def test_configs2_full_size_sse_exact(gpu):
    """8x3x2160x3840 uint8, sigma 4; SSE exact, PSNR consistent."""
    shape = (8, 3, 2160, 3840)
    torch.manual_seed(0)
    g = torch.Generator(device=gpu)
    g.manual_seed(2)
    ta = torch.randint(0, 256, shape, dtype=torch.uint8, device=gpu, generator=g)
    noise = torch.round(torch.randn(shape, device=gpu, generator=g) * 4.0)
    tb = (ta.to(torch.int16) + noise.to(torch.int16)).clamp(0, 255).to(torch.uint8)
    del noise
    per = fa.mse(ta, tb, reduction="none").cpu().numpy()
    a, b = ta.cpu().numpy(), tb.cpu().numpy()
    sse = ref.sse_u8(a, b, per_image=True)
    n = a[0].size
    assert np.array_equal(per, sse.astype(np.float64) / float(n))
    total = float(fa.mse(ta, tb))
    assert total == float(int(sse.sum())) / float(n * 8)
    p = float(fa.psnr(ta, tb, data_range=255.0))
    assert abs(p - (10 * math.log10(255.0 ** 2) - 10 * math.log10(total))) < 1e-12
    assert np.array_equal(fa.l1(ta, tb, reduction="none").cpu().numpy(),
                          ref.sad_u8(a, b, per_image=True).astype(np.float64) / float(n))


@pytest.mark.parametrize("shape", [(2, 1, 2048, 2048),   # 2^22 per image: S == U strides
                                   (3, 3, 1100, 1300),   # S = 5: a round straddles two images
                                   (5, 3, 1080, 1920)])  # 1080p RGB frames
def test_sweep_u8_exact(gpu, shape):
    """Images of >= 2^22 elements take the one-workgroup-per-CU sweep; its
    per-wave partials and image edges keep the integer sums exact."""
    a, b = u8_pair(shape, 6.0, seed=shape[2])
    ta, tb = _t(a, gpu), _t(b, gpu)
    assert np.array_equal(fa.mse(ta, tb, reduction="none").cpu().numpy(), ref.mse(a, b, "none"))
    assert float(fa.mse(ta, tb)) == ref.mse(a, b)
    assert np.array_equal(fa.l1(ta, tb, reduction="none").cpu().numpy(), ref.l1(a, b, "none"))
    p = fa.psnr(ta, tb, data_range=255.0, reduction="none").cpu().numpy()
    assert np.allclose(p, ref.psnr(a, b, 255.0, "none"), rtol=1e-12, atol=0)
    for got, want in ((fa.charbonnier(ta, tb, eps=1e-3, reduction="none"),
                       ref.charbonnier(a, b, 1e-3, "none")),
                      (fa.huber(ta, tb, delta=4.0, reduction="none"), ref.huber(a, b, 4.0, "none"))):
        assert np.allclose(got.cpu().numpy(), want, rtol=1e-6, atol=0)


def test_sweep_fallbacks_exact(gpu):
    """Large images the sweep does not take -- a base off 16-byte alignment,
    or an element count that is not whole 16-byte vectors -- run the per-image
    grid with the sweep's workspace and stay exact."""
    a, b = u8_pair((2, 1, 2049, 2051), 7.0, seed=11)   # 4202499 per image: not whole vectors
    ta, tb = _t(a, gpu), _t(b, gpu)
    assert np.array_equal(fa.mse(ta, tb, reduction="none").cpu().numpy(), ref.mse(a, b, "none"))
    assert np.array_equal(fa.l1(ta, tb, reduction="none").cpu().numpy(), ref.l1(a, b, "none"))
    n = 2 * 2048 * 2048
    base_a, base_b = u8_pair((1, n + 16), 7.0, seed=12)
    for off in (1, 4, 8):
        x = _t(base_a[0], gpu)[off:off + n].view(2, 1, 2048, 2048)
        y = _t(base_b[0], gpu)[off:off + n].view(2, 1, 2048, 2048)
        xa = base_a[0, off:off + n].reshape(2, 1, 2048, 2048)
        yb = base_b[0, off:off + n].reshape(2, 1, 2048, 2048)
        assert np.array_equal(fa.mse(x, y, reduction="none").cpu().numpy(), ref.mse(xa, yb, "none"))
        assert float(fa.l1(x, y)) == ref.l1(xa, yb)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_sweep_float_dtypes(gpu, dt):
    a, b = u8_pair((2, 1, 2048, 2560), 12.0, seed=5)
    xa = torch.from_numpy(a.astype(np.float64) / 255.0).to(dt)
    xb = torch.from_numpy(b.astype(np.float64) / 255.0).to(dt)
    a64, b64 = xa.double().numpy(), xb.double().numpy()
    ta, tb = xa.to(gpu), xb.to(gpu)
    cases = [
        (fa.mse(ta, tb, reduction="none"), ref.mse(a64, b64, "none"), 1e-12),
        (fa.l1(ta, tb, reduction="none"), ref.l1(a64, b64, "none"), 1e-12),
        (fa.huber(ta, tb, delta=0.02, reduction="none"), ref.huber(a64, b64, 0.02, "none"), 1e-12),
        (fa.charbonnier(ta, tb, eps=1e-3, reduction="none"), ref.charbonnier(a64, b64, 1e-3, "none"),
         1e-12 if dt == torch.float64 else 1e-6),
    ]
    for got, want, tol in cases:
        got = got.cpu().numpy()
        assert np.allclose(got, want, rtol=tol, atol=0), (dt, got, want)


@pytest.mark.parametrize("off_a,off_b", [(0, 0), (1, 1), (3, 3), (0, 1), (1, 2), (2, 6),
                                         (4, 8), (5, 13), (15, 0)])
def test_unaligned_views(gpu, off_a, off_b):
    """Contiguous uint8 slices at any byte offset, equal or different between
    the two operands, give the same exact sums (reference
    test_training_metrics.py:423-443)."""
    n = 3 * 64 * 33 + 7
    base_a, base_b = u8_pair((1, n + 32), 20.0, seed=off_a * 31 + off_b)
    ta, tb = _t(base_a[0], gpu), _t(base_b[0], gpu)
    x = ta[off_a:off_a + n]
    y = tb[off_b:off_b + n]
    assert x.is_contiguous() and x.data_ptr() % 16 == (ta.data_ptr() + off_a) % 16
    xs = x.view(1, 1, 1, n)
    ys = y.view(1, 1, 1, n)
    a = base_a[0, off_a:off_a + n][None, None, None]
    b = base_b[0, off_b:off_b + n][None, None, None]
    assert float(fa.mse(xs, ys)) == ref.mse(a, b)
    assert float(fa.l1(xs, ys)) == ref.l1(a, b)
    assert abs(float(fa.huber(xs, ys, delta=3.0)) - ref.huber(a, b, 3.0)) <= 1e-9 * ref.huber(a, b, 3.0)
    # and with several images of odd size, so every image peels its own head
    m = (n - 7) // 3
    x3, y3 = x[: 3 * m].view(3, 1, 1, m), y[: 3 * m].view(3, 1, 1, m)
    a3, b3 = a.reshape(-1)[: 3 * m].reshape(3, 1, 1, m), b.reshape(-1)[: 3 * m].reshape(3, 1, 1, m)
    assert np.array_equal(fa.mse(x3, y3, reduction="none").cpu().numpy(), ref.mse(a3, b3, "none"))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_float_dtypes(gpu, dt):
    a, b = u8_pair((3, 2, 45, 77), 12.0, seed=7)
    xa = torch.from_numpy(a.astype(np.float64) / 255.0).to(dt)
    xb = torch.from_numpy(b.astype(np.float64) / 255.0).to(dt)
    # the oracle sees exactly the values the kernel sees
    a64, b64 = xa.double().numpy(), xb.double().numpy()
    ta, tb = xa.to(gpu), xb.to(gpu)
    for red in ("mean", "none"):
        cases = [
            (fa.mse(ta, tb, reduction=red), ref.mse(a64, b64, red), 1e-12),
            (fa.l1(ta, tb, reduction=red), ref.l1(a64, b64, red), 1e-12),
            (fa.huber(ta, tb, delta=0.02, reduction=red), ref.huber(a64, b64, 0.02, red), 1e-12),
            (fa.charbonnier(ta, tb, eps=1e-3, reduction=red), ref.charbonnier(a64, b64, 1e-3, red),
             1e-12 if dt == torch.float64 else 1e-6),
        ]
        for got, want, tol in cases:
            got, want = got.cpu().numpy(), np.asarray(want)
            assert np.allclose(got, want, rtol=tol, atol=0), (dt, red, got, want)


def test_u8_float_terms(gpu):
    a, b = u8_pair((2, 3, 200, 232), 9.0, seed=3)
    ta, tb = _t(a, gpu), _t(b, gpu)
    for eps in (1e-3, 3.0):
        got = float(fa.charbonnier(ta, tb, eps=eps))
        want = ref.charbonnier(a, b, eps)
        assert abs(got - want) <= 1e-6 * want
    for delta in (1.0, 4.0, 17.0):
        got = float(fa.huber(ta, tb, delta=delta))
        want = ref.huber(a, b, delta)
        assert abs(got - want) <= 1e-6 * want


def test_float64_not_narrowed(gpu):
    """A 1e-6 residual on float64 input has no float32 answer
    (reference test_training_metrics.py:446-463)."""
    x = torch.full((1, 1, 64, 64), 100.0, dtype=torch.float64, device=gpu)
    y = x + 1e-6
    assert abs(float(fa.mse(x, y)) - 1e-12) <= 1e-3 * 1e-12
    assert abs(float(fa.huber(x, y)) - 5e-13) <= 1e-3 * 5e-13
    assert abs(float(fa.l1(x, y)) - 1e-6) <= 1e-3 * 1e-6
    assert abs(float(fa.charbonnier(x, y, eps=0.0)) - 1e-6) <= 1e-3 * 1e-6


def test_identities_and_reductions(gpu):
    x = torch.randint(0, 256, (2, 3, 64, 64), dtype=torch.uint8, device=gpu)
    y = torch.randint(0, 256, (2, 3, 64, 64), dtype=torch.uint8, device=gpu)
    assert float(fa.mse(x, x)) == 0.0
    assert float(fa.psnr(x, x, data_range=255.0)) == float("inf")
    assert float(fa.l1(x, x)) == 0.0 and float(fa.huber(x, x)) == 0.0
    assert abs(float(fa.charbonnier(x, x, eps=0.25)) - 0.25) < 1e-9
    for fn in (fa.mse, fa.l1, fa.charbonnier, fa.huber):
        per = fn(x, y, reduction="none")
        assert per.shape == (2,)
        assert abs(float(per.mean()) - float(fn(x, y))) < 1e-9 * max(1.0, float(fn(x, y)))
    assert fa.psnr(x, y, reduction="none").shape == (2,)
    m = float(fa.mse(x, y))
    assert abs(float(fa.psnr(x, y, data_range=255.0)) - 10 * math.log10(255.0 ** 2 / m)) < 1e-9


def test_luma_and_crop(gpu):
    rng = np.random.default_rng(12)
    a = rng.integers(0, 256, (3, 140, 176)).astype(np.float64)
    b = np.clip(a + 9.0 * rng.standard_normal(a.shape), 0, 255).round()
    ta = torch.from_numpy(a.astype(np.uint8))[None].to(gpu)
    tb = torch.from_numpy(b.astype(np.uint8))[None].to(gpu)
    for mode in ("bt601", "bt709", "matlab"):
        for cb in (0, 4):
            ya = ref.crop(ref.rgb_to_luma(a[None], mode), cb)
            yb = ref.crop(ref.rgb_to_luma(b[None], mode), cb)
            got = float(fa.psnr(ta, tb, data_range=255.0, luma=mode, crop_border=cb))
            assert abs(got - float(ref.psnr(ya, yb, 255.0))) < 1e-10
            want = ref.mse(ya, yb)
            assert abs(float(fa.mse(ta, tb, luma=mode, crop_border=cb)) - want) <= 1e-12 * want
    # an integer crop stays exact
    got = float(fa.mse(ta, tb, crop_border=3))
    assert got == ref.mse(ref.crop(a[None].astype(np.uint8), 3), ref.crop(b[None].astype(np.uint8), 3))


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("cb", [0, 3, 4])
def test_luma_formed_in_kernel(gpu, dt, cb):
    """fa_gpu_pixel_reduce_ex: the luma difference kr dR + kg dG + kb dB in
    float64, crops read in place, every op, against the float64 oracle."""
    a, b = u8_pair((2, 3, 70, 100), 10.0, seed=cb + 7)
    x, y = torch.from_numpy(a).to(gpu, dt), torch.from_numpy(b).to(gpu, dt)
    for mode in ("bt601", "bt709", "matlab"):
        la = ref.crop(ref.rgb_to_luma(a.astype(np.float64), mode), cb)
        lb = ref.crop(ref.rgb_to_luma(b.astype(np.float64), mode), cb)
        kw = dict(luma=mode, crop_border=cb, reduction="none")
        for fn, want in ((fa.mse, ref.mse(la, lb, "none")), (fa.l1, ref.l1(la, lb, "none")),
                         (fa.charbonnier, ref.charbonnier(la, lb, reduction="none")),
                         (fa.huber, ref.huber(la, lb, reduction="none"))):
            got = fn(x, y, **kw).cpu().numpy()
            assert np.all(np.abs(got - want) <= 1e-12 * np.abs(want)), (fn.__name__, mode)
        gp = fa.psnr(x, y, data_range=255.0, **kw).cpu().numpy()
        assert np.all(np.abs(gp - ref.psnr(la, lb, 255.0, "none")) < 1e-10)


@pytest.mark.parametrize("cb", [1, 2, 3, 4, 8])
def test_crop_read_in_place_exact(gpu, cb):
    """uint8 crops stay bit-exact: borders 4 and 8 keep rows 4-byte aligned
    (dword path), 1 / 2 / 3 do not (byte path)."""
    a, b = u8_pair((3, 3, 60, 100), 12.0, seed=cb)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    ca, cbb = ref.crop(a, cb), ref.crop(b, cb)
    got = fa.mse(x, y, crop_border=cb, reduction="none").cpu().numpy()
    assert np.array_equal(got, ref.mse(ca, cbb, "none"))
    got = fa.l1(x, y, crop_border=cb, reduction="none").cpu().numpy()
    assert np.array_equal(got, ref.l1(ca, cbb, "none"))
    assert float(fa.mse(x, y, crop_border=cb)) == ref.mse(ca, cbb)
    # float terms on the byte / dword paths
    got = fa.huber(x, y, crop_border=cb, reduction="none").cpu().numpy()
    want = ref.huber(ca.astype(np.float64), cbb.astype(np.float64), reduction="none")
    assert np.all(np.abs(got - want) <= 1e-9 * np.abs(want))
    got = fa.charbonnier(x, y, eps=0.5, crop_border=cb, reduction="none").cpu().numpy()
    want = ref.charbonnier(ca.astype(np.float64), cbb.astype(np.float64), 0.5, reduction="none")
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want))


@pytest.mark.parametrize("cb", [0, 1, 2, 4])
def test_crop_wide_rows(gpu, cb):
    """Rows wider than one step of the uint8 view kernel (4 KiB), with and
    without luma, an odd row count per image and every byte offset."""
    a, b = u8_pair((2, 3, 13, 4210), 9.0, seed=40 + cb)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    # crop_border=0 on a strided view: a column slice keeps the rows strided
    xs, ys = (x, y) if cb else (x[..., 1:4201], y[..., 1:4201])
    ca = ref.crop(a, cb) if cb else a[..., 1:4201]
    cbb = ref.crop(b, cb) if cb else b[..., 1:4201]
    got = fa.mse(xs, ys, crop_border=cb, reduction="none").cpu().numpy()
    assert np.array_equal(got, ref.mse(ca, cbb, "none"))
    assert np.array_equal(fa.l1(xs, ys, crop_border=cb, reduction="none").cpu().numpy(),
                          ref.l1(ca, cbb, "none"))
    la = ref.rgb_to_luma(ca.astype(np.float64), "bt601")
    lb = ref.rgb_to_luma(cbb.astype(np.float64), "bt601")
    got = fa.mse(xs, ys, luma="bt601", crop_border=cb, reduction="none").cpu().numpy()
    want = ref.mse(la, lb, "none")
    assert np.all(np.abs(got - want) <= 1e-12 * np.abs(want))


@pytest.mark.parametrize("n", [3, 40])
def test_any_workspace_size_exact(gpu, n):
    """fa_gpu_pixel_reduce gives the same exact uint8 sums for any bpi a caller
    passes: the sweep's own (one workgroup per 8 slots, per-workgroup partials
    up to 32 images, per-wave beyond), multiples of 8 that make a smaller or
    larger sweep, and sizes that take the per-image grid."""
    from frame_analytics_amd import backend

    a, b = u8_pair((n, 1, 2048, 2048), 5.0, seed=n)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = a[0].size
    want = ref.mse(a, b, "none")
    stream = torch.cuda.current_stream().cuda_stream
    for bpi in (backend.workspace_slots("pixel", n, per, 0), 8, 64, 4096, 1, 7, 255, 1000):
        part = torch.empty((n, bpi), dtype=torch.float64, device=gpu)
        out = torch.empty(n, dtype=torch.float64, device=gpu)
        rc = backend.call_gpu("fa_gpu_pixel_reduce", x.data_ptr(), y.data_ptr(), 0, n, per, 0,
                              0.0, -1e300, part.data_ptr(), bpi, out.data_ptr(), None, None,
                              None, 0, stream)
        assert rc == 0, (bpi, rc)
        assert np.array_equal(out.cpu().numpy(), want), bpi


def _reduce(name, x, y, op, n, per, bpi, acc, sinks, stream):
    from frame_analytics_amd import backend

    part = torch.empty((n, bpi), dtype=torch.float64, device=x.device)
    args = [x.data_ptr(), y.data_ptr(), 0, n, per, op, 0.0,
            10.0 * math.log10(255.0 ** 2), part.data_ptr(), bpi]
    if name == "fa_gpu_pixel_reduce_once":
        args.append(None if acc is None else acc.data_ptr())
    rc = backend.call_gpu(name, *args, *[s.data_ptr() for s in sinks], 0, stream)
    assert rc == 0, (name, n, per, bpi, rc)


@pytest.mark.parametrize("n,hw,bpis", [
    (1, (2048, 2048), (None, 16, 64, 65536, 1000)),
    (5, (2048, 2048), (None, 16, 4080)),
    (32, (2048, 2048), (None,)),            # the largest batch the one-launch form takes
    (33, (2048, 2048), (None,)),            # beyond it: two launches, acc untouched
    (32, (64, 1024), (16, 32)),             # small images, few workgroups
    (7, (1100, 1300), (None, 48)),          # a round straddles two images
])
def test_single_launch_finish_matches_two_launches(gpu, n, hw, bpis):
    """fa_gpu_pixel_reduce_once: the exact uint8 MSE / L1 sums finished inside
    the sweep by returning atomics give the same per-image and total values,
    and the same dB, bit for bit, as fa_gpu_pixel_reduce (itself exact against
    the oracle's integer sums), for workspace shapes that take the one-launch
    form and ones that do not; the accumulator is zero after every call,
    including a second, smaller call on the same buffer."""
    from frame_analytics_amd import backend

    g = torch.Generator(device=gpu)
    g.manual_seed(n * 7 + hw[0])
    shape = (n, 1) + hw
    x = torch.randint(0, 256, shape, dtype=torch.uint8, device=gpu, generator=g)
    y = (x.to(torch.int16) + torch.randint(-9, 10, shape, dtype=torch.int16, device=gpu,
                                           generator=g)).clamp(0, 255).to(torch.uint8)
    per = hw[0] * hw[1]
    stream = torch.cuda.current_stream().cuda_stream
    acc = torch.zeros(backend._ACC_WORDS["pixel"], dtype=torch.int64, device=gpu)
    a_np, b_np = x.cpu().numpy(), y.cpu().numpy()
    for op, isum in ((0, ref.sse_u8(a_np, b_np, per_image=True)),
                     (1, ref.sad_u8(a_np, b_np, per_image=True))):
        isum = [int(v) for v in isum]
        want = np.asarray(isum, dtype=np.float64) / float(per)
        for bpi in bpis:
            bpi = backend.workspace_slots("pixel", n, per, 0) if bpi is None else bpi
            for m in (n, max(1, n - 2)):  # a second, smaller call on the same acc
                xs, ys = x[:m], y[:m]
                two = [torch.full((m,), -1.0, dtype=torch.float64, device=gpu),
                       torch.full((), -1.0, dtype=torch.float64, device=gpu),
                       torch.full((m,), -1.0, dtype=torch.float64, device=gpu),
                       torch.full((), -1.0, dtype=torch.float64, device=gpu)]
                one = [t.clone() for t in two]
                _reduce("fa_gpu_pixel_reduce", xs, ys, op, m, per, bpi, None, two, stream)
                _reduce("fa_gpu_pixel_reduce_once", xs, ys, op, m, per, bpi, acc, one, stream)
                for t1, t2 in zip(one, two):
                    assert torch.equal(t1, t2), (op, bpi, m, t1, t2)
                assert np.array_equal(one[0].cpu().numpy(), want[:m]), (op, bpi, m)
                assert float(one[1]) == float(sum(isum[:m])) / float(per * m)
                assert not bool(acc.any()), (op, bpi, m, acc.nonzero())
            # only the total wanted, then only per-image values: the image
            # finishers still run, and the total word is left zero either way
            for pick in ((1,), (0,), (3,), (2,)):
                outs = [torch.full((n,) if i % 2 == 0 else (), -1.0, dtype=torch.float64,
                                   device=gpu) for i in range(4)]
                sinks = [outs[i] if i in pick else None for i in range(4)]
                part = torch.empty((n, bpi), dtype=torch.float64, device=gpu)
                rc = backend.call_gpu(
                    "fa_gpu_pixel_reduce_once", x.data_ptr(), y.data_ptr(), 0, n, per, op, 0.0,
                    10.0 * math.log10(255.0 ** 2), part.data_ptr(), bpi, acc.data_ptr(),
                    *[None if s is None else s.data_ptr() for s in sinks], 0, stream)
                assert rc == 0
                if 0 in pick:
                    assert np.array_equal(outs[0].cpu().numpy(), want)
                if 1 in pick:
                    assert float(outs[1]) == float(sum(isum)) / float(per * n)
                assert not bool(acc.any()), (op, bpi, pick)


def test_single_launch_finish_per_stream(gpu):
    """fa.mse / fa.psnr on two streams at once: each stream has its own
    accumulator, so interleaved calls stay exact."""
    from frame_analytics_amd import backend

    a, b = u8_pair((3, 1, 2048, 2048), 7.0, seed=11)
    c, d = u8_pair((2, 3, 1100, 1300), 3.0, seed=12)
    ta, tb, tc, td = (_t(v, gpu) for v in (a, b, c, d))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for _ in range(4):
        with torch.cuda.stream(s1):
            outs.append(("ab", fa.mse(ta, tb, reduction="none")))
        with torch.cuda.stream(s2):
            outs.append(("cd", fa.mse(tc, td, reduction="none")))
    torch.cuda.synchronize()
    for key, o in outs:
        want = ref.mse(a, b, "none") if key == "ab" else ref.mse(c, d, "none")
        assert np.array_equal(o.cpu().numpy(), want), key
    keys = [k for k in backend._stream_acc
            if k[0] == "pixel" and k[2] in (s1.cuda_stream, s2.cuda_stream)]
    assert len(keys) == 2
    for k in keys:
        assert not bool(backend._stream_acc[k].any())


def test_single_launch_without_workspace(gpu):
    """fa_gpu_pixel_reduce_once with a null `partial`: where the call finishes
    in the sweep the workspace is not read and the values are the same; where
    it cannot (a workspace shape the sweep does not take, an op without exact
    sums) the call returns FA_E_ARG and writes nothing."""
    from frame_analytics_amd import backend

    a, b = u8_pair((3, 1, 2048, 2048), 6.0, seed=31)
    x, y = _t(a, gpu), _t(b, gpu)
    n, per = 3, 2048 * 2048
    st = torch.cuda.current_stream().cuda_stream
    acc = torch.zeros(backend._ACC_WORDS["pixel"], dtype=torch.int64, device=gpu)
    bias = 10.0 * math.log10(255.0 ** 2)
    bpi = backend.workspace_slots("pixel", n, per, 0)
    for op, bp, ok in ((0, bpi, True), (1, bpi, True), (0, 1000, False), (2, bpi, False)):
        out = torch.full((n,), -1.0, dtype=torch.float64, device=gpu)
        rc = backend.call_gpu("fa_gpu_pixel_reduce_once", x.data_ptr(), y.data_ptr(), 0, n, per,
                              op, 1e-6, bias, None, bp, acc.data_ptr(), out.data_ptr(), None,
                              None, None, 0, st)
        torch.cuda.synchronize()
        if ok:
            assert rc == 0
            want = ref.mse(a, b, "none") if op == 0 else ref.l1(a, b, "none")
            assert np.array_equal(out.cpu().numpy(), want)
        else:
            assert rc == 5 and bool((out == -1.0).all()), (op, bp, rc)
        assert not bool(acc.any())
