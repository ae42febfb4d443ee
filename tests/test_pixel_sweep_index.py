"""CPU check of the pixel sweep's indexing (pix_sweep_kernel in
frame_analytics_amd/csrc/fa_pixel.hip), for launch shapes and batch sizes the
GPU tests do not all reach.

The model steps every lane of the grid through the kernel's rounds with the
kernel's own decisions: the wave-uniform fast / edge / end paths, the per-lane
image split and the emit loop.  It checks what a GPU run cannot show safely:
every load lies inside the batch, every (image, wave) partial is written
exactly once, and each image's partials hold exactly that image's vectors (each
vector carries its own index as its value, so a misrouted or repeated vector
changes a sum).
"""

from __future__ import annotations

import numpy as np
import pytest

WAVE = 64


def simulate_sweep(nv: int, n_images: int, G: int, NT: int, U: int):
    """Returns (per-image sums of vector indices over the wave partials,
    number of writes per slot, largest vector index loaded)."""
    assert nv >= U * G * NT, "the host launches the sweep only when a round spans <= one image"
    total = nv * n_images
    gs = G * NT
    t0 = np.arange(G * NT, dtype=np.int64)
    w0 = t0 - (t0 % WAVE)
    nwaves = G * NT // WAVE
    wave_of = t0 // WAVE
    img = np.zeros(nwaves, np.int64)
    edge = np.full(nwaves, nv, np.int64)
    cur = np.zeros(G * NT, np.int64)
    nxt = np.zeros(G * NT, np.int64)
    sums = np.zeros((n_images, nwaves), np.int64)
    writes = np.zeros((n_images, nwaves), np.int64)
    max_load = -1
    base = 0
    while True:
        active_w = img < n_images
        if not active_w.any():
            break
        act = active_w[wave_of]
        e = edge[wave_of]
        last = base + (U - 1) * gs + w0 + (WAVE - 1)
        fast = act & (last < e)
        edgep = act & ~fast & (last < total)
        endp = act & ~fast & ~edgep
        for u in range(U):
            v = base + u * gs + t0
            loads = fast | edgep | (endp & (v < total))
            if loads.any():
                max_load = max(max_load, int(v[loads].max()))
            hi = v >= e
            to_cur = loads & (fast | ~hi)
            to_nxt = loads & ~fast & hi
            cur[to_cur] += v[to_cur]
            nxt[to_nxt] += v[to_nxt]
        nxt_pos = base + U * gs + w0[::WAVE]  # per wave
        while True:
            em = (img < n_images) & (nxt_pos >= edge)
            if not em.any():
                break
            lanes = em[wave_of]
            part = np.zeros(nwaves, np.int64)
            np.add.at(part, wave_of[lanes], cur[lanes])
            ws = np.nonzero(em)[0]
            sums[img[ws], ws] += part[ws]
            writes[img[ws], ws] += 1
            cur[lanes] = nxt[lanes]
            nxt[lanes] = 0
            img[em] += 1
            edge[em] += nv
        base += U * gs
    return sums.sum(axis=1), writes, max_load


CASES = [
    # (nv, n_images, G, NT, U)
    (1_555_200, 8, 256, 512, 2),   # configs[2] on a 256-CU part, the large-batch shape
    (388_800, 8, 256, 1024, 1),    # configs[4] 8x3x1080x1920 uint8, the many-wave shape
    (262_144, 3, 256, 1024, 1),    # many-wave shape, exactly one round per image
    (300_001, 33, 256, 1024, 1),   # many-wave shape past the LDS image limit
    (1_555_200, 8, 256, 256, 4),   # the 4 x 256 launch shape
    (1_555_200, 8, 256, 512, 4),   # 4 x 512: a short last round, waves finish a round early
    (268_125, 3, 256, 256, 4),     # 3x3x1100x1300 uint8
    (388_800, 8, 256, 256, 4),     # 8x3x1080x1920 uint8
    (262_144, 2, 256, 256, 4),     # exactly one round per image
    (262_145, 5, 256, 256, 4),
    (320_001, 7, 304, 256, 4),     # another CU count
    (130_000, 3, 80, 512, 3),
    (65_536, 4, 64, 256, 4),
]


@pytest.mark.parametrize("nv,n_images,G,NT,U", CASES)
def test_sweep_indexing(nv, n_images, G, NT, U):
    sums, writes, max_load = simulate_sweep(nv, n_images, G, NT, U)
    total = nv * n_images
    assert max_load == total - 1  # every load inside the batch, the last vector read
    assert (writes == 1).all()    # each (image, wave) partial written once
    i = np.arange(n_images, dtype=np.int64)
    want = nv * (i * nv) + nv * (nv - 1) // 2  # sum of the image's vector indices
    assert np.array_equal(sums, want)
