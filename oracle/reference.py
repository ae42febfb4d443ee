"""float64 NumPy oracle for the fused metric path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  Nothing in
``frame_analytics_amd`` imports it.

Each function restates, from the papers and the reference's own float64
transcription, what the reference computes (citations are into
NevermindNilas/frame_analytics).  Arrays are float64 throughout; uint8 MSE/L1
are exact integer sums.

How each function is pinned (see tests/test_oracle.py):
  * gaussian / valid correlation: direct 121-tap 2-D correlation, scipy's
    correlate2d, fspecial closed form, window sums to 1
  * mse / psnr / l1 / charbonnier / huber: brute-force int64 sums, torch's
    huber_loss / l1_loss, identities (psnr(x,x)=inf, charbonnier(x,x)=eps)
  * ssim / cs: identity ssim(x,x)=1, scipy cross-check, the reference's own
    CPU C++ (oracle/_ref, built from the reference sources) at its 5e-6 gate
  * ms_ssim: single-scale special cases reduce to ssim / cs, avg-pool via torch,
    the reference CPU C++ per-scale primitive, the reference's own
    "channels averaged after the product" case (two 1-channel values against
    one 2-channel call, with the channel-mean-first variant as a negative
    control), weights (0,0,0,0,1) against ssim of the pair pooled four times
    by torch, and the clamp on an anti-correlated pair (exactly 0)
  * ms_ssim gradient: float64 central differences of ms_ssim
  * gmsd: identity, the reference CPU C++ gmsd, torch conv2d Prewitt;
    gmsd_stats_hp: gmsd_stats at ordinary noise, a 40-digit decimal brute force
  * ssim gradient: float64 central differences and float64 torch autograd
  * gms / gmsd gradient: float64 central differences of gmsd_stats
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np

MS_SSIM_WEIGHTS = (0.0448, 0.2856, 0.3001, 0.2363, 0.1333)  # reference.py:69

# (r, g, b, offset as a fraction of L) -- reference.py:81-85
LUMA_COEFFS = {
    "bt601": (0.299, 0.587, 0.114, 0.0),
    "bt709": (0.2126, 0.7152, 0.0722, 0.0),
    "matlab": (65.481 / 255.0, 128.553 / 255.0, 24.966 / 255.0, 16.0 / 255.0),
}


# --------------------------------------------------------------------------- #
# windows and correlation
# --------------------------------------------------------------------------- #


def gaussian_window_2d(win_size: int = 11, sigma: float = 1.5) -> np.ndarray:
    """MATLAB ``fspecial('gaussian')``: exp(-(i^2+j^2)/(2 sigma^2)), entries
    below eps*max zeroed, normalised to sum 1 (reference.py:88-99)."""
    c = np.arange(win_size, dtype=np.float64) - (win_size - 1) / 2.0
    g = np.exp(-(c[:, None] ** 2 + c[None, :] ** 2) / (2.0 * sigma * sigma))
    g[g < np.finfo(np.float64).eps * g.max()] = 0.0
    return g / g.sum()


def gaussian_window_1d(win_size: int = 11, sigma: float = 1.5) -> np.ndarray:
    """1-D factor of the window, normalised in float64 (functional.py:397-420)."""
    c = np.arange(win_size, dtype=np.float64) - (win_size - 1) / 2.0
    g = np.exp(-(c * c) / (2.0 * sigma * sigma))
    return g / g.sum()


def valid_correlate2d(img: np.ndarray, k: np.ndarray) -> np.ndarray:
    """Direct 'valid' 2-D correlation over the last two axes (MATLAB filter2,
    reference.py:102-115)."""
    kh, kw = k.shape
    h, w = img.shape[-2:]
    oh, ow = h - kh + 1, w - kw + 1
    if oh <= 0 or ow <= 0:
        raise ValueError(f"image {img.shape} smaller than window {k.shape}")
    out = np.zeros(img.shape[:-2] + (oh, ow), dtype=np.float64)
    for i in range(kh):
        for j in range(kw):
            if k[i, j] != 0.0:
                out += k[i, j] * img[..., i:i + oh, j:j + ow]
    return out


def separable_valid(img: np.ndarray, w: np.ndarray) -> np.ndarray:
    """'valid' correlation with the outer product w w^T, as two 1-D passes over
    the last two axes.  Equal to valid_correlate2d(img, outer(w, w)) up to
    float64 rounding."""
    k = w.size
    h, wd = img.shape[-2:]
    oh, ow = h - k + 1, wd - k + 1
    if oh <= 0 or ow <= 0:
        raise ValueError(f"image {img.shape} smaller than window {k}")
    t = np.zeros(img.shape[:-1] + (ow,), dtype=np.float64)
    for j in range(k):
        t += w[j] * img[..., :, j:j + ow]
    out = np.zeros(img.shape[:-2] + (oh, ow), dtype=np.float64)
    for i in range(k):
        out += w[i] * t[..., i:i + oh, :]
    return out


# --------------------------------------------------------------------------- #
# SSIM
# --------------------------------------------------------------------------- #


def ssim_maps(x, y, data_range=255.0, win_size=11, sigma=1.5, K1=0.01, K2=0.03):
    """``(ssim_map, cs_map)`` over the last two axes (reference.py:130-158):
    mu = w*x, sigma_xx = w*x^2 - mu_x^2, sigma_xy = w*xy - mu_x mu_y,
    cs = (2 sxy + C2)/(sxx + syy + C2), l = (2 mx my + C1)/(mx^2 + my^2 + C1)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    if x.shape != y.shape:
        raise ValueError(f"shape mismatch: {x.shape} vs {y.shape}")
    w = gaussian_window_1d(win_size, sigma)
    C1 = (K1 * data_range) ** 2
    C2 = (K2 * data_range) ** 2
    mx = separable_valid(x, w)
    my = separable_valid(y, w)
    sxx = separable_valid(x * x, w) - mx * mx
    syy = separable_valid(y * y, w) - my * my
    sxy = separable_valid(x * y, w) - mx * my
    cs = (2.0 * sxy + C2) / (sxx + syy + C2)
    lum = (2.0 * mx * my + C1) / (mx * mx + my * my + C1)
    return lum * cs, cs


def ssim(x, y, data_range=255.0, win_size=11, sigma=1.5, K=(0.01, 0.03),
         reduction="mean", return_map=False):
    """fa.ssim on (N, C, H, W): map mean per image, batch mean of those
    (functional.py:589-689; reference.py:161-175 per plane)."""
    smap, _ = ssim_maps(x, y, data_range, win_size, sigma, K[0], K[1])
    if return_map:
        return smap
    per_image = smap.reshape(smap.shape[0], -1).mean(axis=1)
    return per_image if reduction == "none" else float(per_image.mean())


# --------------------------------------------------------------------------- #
# MSE / PSNR / pixel losses
# --------------------------------------------------------------------------- #


def _u8_pair(x, y) -> bool:
    return np.asarray(x).dtype == np.uint8 and np.asarray(y).dtype == np.uint8


def sse_u8(x: np.ndarray, y: np.ndarray, per_image: bool = False, chunk: int = 1 << 24):
    """Exact integer sum of squared differences of uint8 arrays, per leading
    index when ``per_image`` (chunked to bound memory)."""
    a = np.ascontiguousarray(x).reshape(x.shape[0], -1)
    b = np.ascontiguousarray(y).reshape(y.shape[0], -1)
    out = np.zeros(a.shape[0], dtype=np.int64)
    for i in range(a.shape[0]):
        for s in range(0, a.shape[1], chunk):
            d = a[i, s:s + chunk].astype(np.int32) - b[i, s:s + chunk].astype(np.int32)
            out[i] += int(np.dot(d.astype(np.int64), d.astype(np.int64)))
    return out if per_image else int(out.sum())


def sad_u8(x: np.ndarray, y: np.ndarray, per_image: bool = False, chunk: int = 1 << 24):
    """Exact integer sum of absolute differences of uint8 arrays."""
    a = np.ascontiguousarray(x).reshape(x.shape[0], -1)
    b = np.ascontiguousarray(y).reshape(y.shape[0], -1)
    out = np.zeros(a.shape[0], dtype=np.int64)
    for i in range(a.shape[0]):
        for s in range(0, a.shape[1], chunk):
            d = a[i, s:s + chunk].astype(np.int32) - b[i, s:s + chunk].astype(np.int32)
            out[i] += int(np.abs(d).sum(dtype=np.int64))
    return out if per_image else int(out.sum())


def mse(x, y, reduction="mean"):
    """mean((x-y)^2) (reference.py:118-120); exact for uint8 (integer SSE
    divided once by the count)."""
    n = np.asarray(x).shape[0]
    per = np.asarray(x).size // n
    if _u8_pair(x, y):
        s = sse_u8(x, y, per_image=True)
        if reduction == "none":
            return s.astype(np.float64) / float(per)
        return float(int(s.sum())) / float(per * n)
    d = np.asarray(x, np.float64) - np.asarray(y, np.float64)
    sq = (d * d).reshape(n, -1)
    if reduction == "none":
        return sq.sum(axis=1) / per
    return float(sq.sum() / sq.size)


def psnr(x, y, data_range=255.0, reduction="mean"):
    """10 log10(L^2 / mse) dB, +inf for mse 0 (reference.py:123-127), written
    as 10 log10(L^2) - 10 log10(mse) like functional.py:370,387."""
    m = mse(x, y, reduction)
    bias = 10.0 * np.log10(data_range * data_range)
    with np.errstate(divide="ignore"):
        return bias - 10.0 * np.log10(m)


def _pixel(x, y, term, reduction):
    d = np.asarray(x, np.float64) - np.asarray(y, np.float64)
    t = term(d).reshape(d.shape[0], -1)
    return t.mean(axis=1) if reduction == "none" else float(t.sum() / t.size)


def l1(x, y, reduction="mean"):
    """mean |x - y| (reference.py:183-184); exact for uint8."""
    if _u8_pair(x, y):
        n = np.asarray(x).shape[0]
        per = np.asarray(x).size // n
        s = sad_u8(x, y, per_image=True)
        if reduction == "none":
            return s.astype(np.float64) / float(per)
        return float(int(s.sum())) / float(per * n)
    return _pixel(x, y, np.abs, reduction)


def charbonnier(x, y, eps=1e-3, reduction="mean"):
    """mean sqrt(d^2 + eps^2) (reference.py:187-195)."""
    e2 = float(eps) ** 2
    return _pixel(x, y, lambda d: np.sqrt(d * d + e2), reduction)


def huber(x, y, delta=1.0, reduction="mean"):
    """0.5 d^2 inside delta, delta(|d| - delta/2) outside (reference.py:198-204)."""
    dl = float(delta)

    def term(d):
        a = np.abs(d)
        return np.where(a <= dl, 0.5 * a * a, dl * (a - 0.5 * dl))

    return _pixel(x, y, term, reduction)


# --------------------------------------------------------------------------- #
# luma / crop
# --------------------------------------------------------------------------- #


def rgb_to_luma(img, mode="bt601", data_range=255.0):
    """(..., 3, H, W) -> (..., 1, H, W) (reference.py:212-223)."""
    img = np.asarray(img, dtype=np.float64)
    kr, kg, kb, off = LUMA_COEFFS[mode]
    out = kr * img[..., 0, :, :] + kg * img[..., 1, :, :] + kb * img[..., 2, :, :]
    return (out + off * float(data_range))[..., None, :, :]


def crop(img, b):
    if not b:
        return img
    return img[..., b:img.shape[-2] - b, b:img.shape[-1] - b]


# --------------------------------------------------------------------------- #
# MS-SSIM
# --------------------------------------------------------------------------- #


def avg_pool2(x: np.ndarray) -> np.ndarray:
    """Non-overlapping 2x2 mean, odd trailing row/column dropped
    (reference.py:231-241)."""
    h, w = x.shape[-2] // 2 * 2, x.shape[-1] // 2 * 2
    v = np.asarray(x, np.float64)[..., :h, :w]
    return v.reshape(*v.shape[:-2], h // 2, 2, w // 2, 2).mean(axis=(-3, -1))


def ms_ssim_terms(x, y, data_range=255.0, win_size=11, sigma=1.5, K=(0.01, 0.03),
                  scales=5):
    """Per-scale plane means ``[(ssim_s, cs_s)]``, each (N, C) (the native
    primitive at every pyramid level, functional.py:876-887)."""
    cx = np.asarray(x, np.float64)
    cy = np.asarray(y, np.float64)
    out = []
    for i in range(scales):
        if i:
            cx, cy = avg_pool2(cx), avg_pool2(cy)
        s, cs = ssim_maps(cx, cy, data_range, win_size, sigma, K[0], K[1])
        out.append((s.mean(axis=(-2, -1)), cs.mean(axis=(-2, -1))))
    return out


def ms_ssim(x, y, data_range=255.0, win_size=11, sigma=1.5, K=(0.01, 0.03),
            weights: Sequence[float] = MS_SSIM_WEIGHTS, reduction="mean"):
    """prod_j max(cs_j, 0)^w_j with the full SSIM at the coarsest scale, per
    (image, channel); channels averaged after the product, then images
    (reference.py:244-276 per plane; functional.py:897-901 for the batch)."""
    w = list(weights)
    terms = ms_ssim_terms(x, y, data_range, win_size, sigma, K, len(w))
    per_plane = np.ones_like(terms[0][0])
    for i, wi in enumerate(w):
        v = terms[i][0] if i == len(w) - 1 else terms[i][1]
        per_plane = per_plane * np.maximum(v, 0.0) ** wi
    per_image = per_plane.mean(axis=1)
    return per_image if reduction == "none" else float(per_image.mean())


# --------------------------------------------------------------------------- #
# GMSD
# --------------------------------------------------------------------------- #

PREWITT_X = np.array([[1.0, 0.0, -1.0]] * 3) / 3.0  # reference.py:284
PREWITT_Y = PREWITT_X.T.copy()


def gms_map(x, y, data_range=255.0, T=None, downsample=True, eps=None):
    """q = (2 g1 g2 + T)/(g1^2 + g2^2 + T), g = sqrt(gx^2 + gy^2 + eps), valid
    Prewitt, optional 2x2 mean downsample (reference.py:288-335 with the
    functional.py:984-985 defaults T = 170 (L/255)^2, eps = (1e-6 L)^2)."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    L = float(data_range)
    T = 170.0 * (L / 255.0) ** 2 if T is None else float(T)
    eps = (1e-6 * L) ** 2 if eps is None else float(eps)
    if downsample:
        x, y = avg_pool2(x), avg_pool2(y)
    g1 = np.sqrt(valid_correlate2d(x, PREWITT_X) ** 2 + valid_correlate2d(x, PREWITT_Y) ** 2 + eps)
    g2 = np.sqrt(valid_correlate2d(y, PREWITT_X) ** 2 + valid_correlate2d(y, PREWITT_Y) ** 2 + eps)
    return (2.0 * g1 * g2 + T) / (g1 * g1 + g2 * g2 + T)


def gmsd_stats(x, y, data_range=255.0, T=None, downsample=True, eps=None):
    """Per image (pooled over channels): ``(mean q, population std q)``
    (functional.py:959-971, fa_cuda.cu:1005-1026)."""
    q = gms_map(x, y, data_range, T, downsample, eps)
    f = q.reshape(q.shape[0], -1)
    m = f.mean(axis=1)
    return m, np.sqrt(((f - m[:, None]) ** 2).mean(axis=1))


def gmsd_stats_hp(x, y, data_range=255.0, T=None, downsample=True, eps=None):
    """The statistics of :func:`gmsd_stats`, evaluated through d = 1 - q in a
    cancellation-free float64 form, for nearly identical images where q sits
    within 1e-9 of 1 and ``gmsd_stats``' own rounding (~1e-16 on q) is no
    longer small against the spread.

    With s = x + y, e = x - y and P the Prewitt response (linear):
    g1 = (Ps + Pe)/2, g2 = (Ps - Pe)/2, g1^2 - g2^2 = Pxs Pxe + Pys Pye, and
    1 - q = (g1 - g2)^2 / (g1^2 + g2^2 + T) with
    (g1 - g2)^2 = (G1 - G2)^2 / (sqrt G1 + sqrt G2)^2, G = g^2.  The 2x2 mean
    is taken of e itself, not of two rounded means.  Same mathematics as the
    reference's functional.py:959-971; pinned against ``gmsd_stats`` at
    ordinary noise and against a 40-digit decimal brute force."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    L = float(data_range)
    T = 170.0 * (L / 255.0) ** 2 if T is None else float(T)
    eps = (1e-6 * L) ** 2 if eps is None else float(eps)
    s, e = x + y, x - y
    if downsample:
        s, e = avg_pool2(s), avg_pool2(e)
    pxs, pys = valid_correlate2d(s, PREWITT_X), valid_correlate2d(s, PREWITT_Y)
    pxe, pye = valid_correlate2d(e, PREWITT_X), valid_correlate2d(e, PREWITT_Y)
    G1 = 0.25 * ((pxs + pxe) ** 2 + (pys + pye) ** 2) + eps
    G2 = 0.25 * ((pxs - pxe) ** 2 + (pys - pye) ** 2) + eps
    dG = pxs * pxe + pys * pye
    den = (G1 + G2 + 2.0 * np.sqrt(G1 * G2)) * (G1 + G2 + T)
    d = np.divide(dG * dG, den, out=np.zeros_like(den), where=den > 0)
    f = d.reshape(d.shape[0], -1)
    m = f.mean(axis=1)
    return 1.0 - m, np.sqrt(((f - m[:, None]) ** 2).mean(axis=1))


# --------------------------------------------------------------------------- #
# SSIM gradient (closed-form adjoint)
# --------------------------------------------------------------------------- #


def full_correlate_transposed(m: np.ndarray, w: np.ndarray, H: int, W: int) -> np.ndarray:
    """(w^T * m)(q) = sum_p w(q - p) m(p): the adjoint of the valid correlation,
    from the (H-K+1) x (W-K+1) grid back onto H x W with zeros outside."""
    k = w.size
    oh, ow = m.shape[-2:]
    out = np.zeros(m.shape[:-2] + (H, W), dtype=np.float64)
    for i in range(k):
        for j in range(k):
            out[..., i:i + oh, j:j + ow] += w[i] * w[j] * m
    return out


def ssim_mean_grad(x, y, data_range=1.0, win_size=11, sigma=1.5, K=(0.01, 0.03),
                   upstream: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """d L / d x and d L / d y in float64, L = sum(upstream * ssim_map), with
    upstream defaulting to 1/(map size) (the gradient of the batch-mean SSIM).

    dS/dsxy = 2 A1/(B1 B2); dS/dsxx = dS/dsyy = -S/B2;
    dS/dmux = 2 A2/(B1 B2) (my - mx A1/B1); then by the chain rule through
    mu = w*x, sxx = w*x^2 - mu^2, sxy = w*xy - mu_x mu_y:
    dx = 2 x (w^T*b) + y (w^T*c) + w^T*(g dS/dmux - 2 b mx - c my)."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    w = gaussian_window_1d(win_size, sigma)
    C1 = (K[0] * data_range) ** 2
    C2 = (K[1] * data_range) ** 2
    mx = separable_valid(x, w)
    my = separable_valid(y, w)
    sxx = separable_valid(x * x, w) - mx * mx
    syy = separable_valid(y * y, w) - my * my
    sxy = separable_valid(x * y, w) - mx * my
    A1 = 2 * mx * my + C1
    A2 = 2 * sxy + C2
    B1 = mx * mx + my * my + C1
    B2 = sxx + syy + C2
    S = A1 * A2 / (B1 * B2)
    g = np.full(S.shape, 1.0 / S.size) if upstream is None else np.asarray(upstream, np.float64)
    b = g * (-S / B2)
    c = g * (2 * A1 / (B1 * B2))
    dmux = 2 * A2 / (B1 * B2) * (my - mx * A1 / B1)
    dmuy = 2 * A2 / (B1 * B2) * (mx - my * A1 / B1)
    tx = g * dmux - 2 * b * mx - c * my
    ty = g * dmuy - 2 * b * my - c * mx
    H, W = x.shape[-2:]
    Pb = full_correlate_transposed(b, w, H, W)
    Pc = full_correlate_transposed(c, w, H, W)
    dx = 2 * x * Pb + y * Pc + full_correlate_transposed(tx, w, H, W)
    dy = 2 * y * Pb + x * Pc + full_correlate_transposed(ty, w, H, W)
    return dx, dy


def ssim_cs_map_grad(x, y, g_s, g_cs, data_range=1.0, win_size=11, sigma=1.5,
                     K=(0.01, 0.03)) -> Tuple[np.ndarray, np.ndarray]:
    """d L / d x and d L / d y in float64 for L = sum(g_s * ssim_map + g_cs * cs_map)
    over the last two axes; g_s, g_cs broadcast against the (H-K+1, W-K+1) maps.

    cs = A2/B2 depends on the means only through the variances:
    dcs/dsxy = 2/B2, dcs/dsxx = dcs/dsyy = -cs/B2, no direct mu term.  The
    SSIM part is that of :func:`ssim_mean_grad`; the two share the chain rule
    through mu = w*x, sxx = w*x^2 - mu^2, sxy = w*xy - mu_x mu_y."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    w = gaussian_window_1d(win_size, sigma)
    C1 = (K[0] * data_range) ** 2
    C2 = (K[1] * data_range) ** 2
    mx = separable_valid(x, w)
    my = separable_valid(y, w)
    sxx = separable_valid(x * x, w) - mx * mx
    syy = separable_valid(y * y, w) - my * my
    sxy = separable_valid(x * y, w) - mx * my
    A1 = 2 * mx * my + C1
    A2 = 2 * sxy + C2
    B1 = mx * mx + my * my + C1
    B2 = sxx + syy + C2
    S = A1 * A2 / (B1 * B2)
    cs = A2 / B2
    gs = np.broadcast_to(np.asarray(g_s, np.float64), S.shape)
    gc = np.broadcast_to(np.asarray(g_cs, np.float64), S.shape)
    b = gs * (-S / B2) + gc * (-cs / B2)
    c = gs * (2 * A1 / (B1 * B2)) + gc * (2.0 / B2)
    tx = gs * (2 * A2 / (B1 * B2) * (my - mx * A1 / B1)) - 2 * b * mx - c * my
    ty = gs * (2 * A2 / (B1 * B2) * (mx - my * A1 / B1)) - 2 * b * my - c * mx
    H, W = x.shape[-2:]
    Pb = full_correlate_transposed(b, w, H, W)
    Pc = full_correlate_transposed(c, w, H, W)
    dx = 2 * x * Pb + y * Pc + full_correlate_transposed(tx, w, H, W)
    dy = 2 * y * Pb + x * Pc + full_correlate_transposed(ty, w, H, W)
    return dx, dy


def avg_pool2_adjoint(g: np.ndarray, H: int, W: int) -> np.ndarray:
    """Adjoint of :func:`avg_pool2` onto an H x W plane: a quarter of each
    pooled gradient to every pixel of its 2x2 block, nothing to a dropped odd
    trailing row or column."""
    h, w = g.shape[-2:]
    out = np.zeros(g.shape[:-2] + (H, W), dtype=np.float64)
    out[..., :2 * h, :2 * w] = 0.25 * np.repeat(np.repeat(g, 2, axis=-2), 2, axis=-1)
    return out


def ms_ssim_grad(x, y, data_range=1.0, win_size=11, sigma=1.5, K=(0.01, 0.03),
                 weights: Sequence[float] = MS_SSIM_WEIGHTS,
                 upstream=None) -> Tuple[np.ndarray, np.ndarray]:
    """d L / d x and d L / d y in float64 of L = sum_n u[n] * ms_ssim_n(x, y),
    the per-image MS-SSIM of :func:`ms_ssim` (``upstream`` u; default 1/N,
    the gradient of the batch mean).

    Through the composition of functional.py:887-901: per plane
    P = prod_j max(t_j, 0)^w_j, so dP/dt_j = w_j t_j^(w_j - 1) prod_{k != j}
    max(t_k, 0)^w_k for t_j > 0 and 0 where the clamp holds; the channel
    mean gives each plane u[n]/C; t_j is the plane mean of the cs map (the
    SSIM map at the coarsest scale), so its map-level upstream is
    dP/dt_j / (map size); each level's gradient reaches the level above
    through the 2x2 mean's adjoint."""
    cx = np.asarray(x, np.float64)
    cy = np.asarray(y, np.float64)
    N, C = cx.shape[:2]
    wts = [float(v) for v in weights]
    M = len(wts)
    levels = [(cx, cy)]
    for _ in range(M - 1):
        levels.append((avg_pool2(levels[-1][0]), avg_pool2(levels[-1][1])))
    terms = []
    for j, (lx, ly) in enumerate(levels):
        s, cs = ssim_maps(lx, ly, data_range, win_size, sigma, K[0], K[1])
        terms.append((s if j == M - 1 else cs).mean(axis=(-2, -1)))
    t = np.stack(terms)                       # (M, N, C)
    tc = np.maximum(t, 0.0)
    u = np.full(N, 1.0 / N) if upstream is None else np.asarray(upstream, np.float64)
    gP = np.broadcast_to((u / C)[:, None], (N, C))
    gx = gy = None
    for j in range(M - 1, -1, -1):
        others = np.ones((N, C))
        for k in range(M):
            if k != j:
                others = others * tc[k] ** wts[k]
        with np.errstate(divide="ignore", invalid="ignore"):
            dt = np.where(t[j] > 0, wts[j] * tc[j] ** (wts[j] - 1.0), 0.0) * others * gP
        lx, ly = levels[j]
        npix = (lx.shape[-2] - win_size + 1) * (lx.shape[-1] - win_size + 1)
        g = (dt / npix)[..., None, None]
        zero = np.zeros_like(g)
        dlx, dly = ssim_cs_map_grad(lx, ly, g if j == M - 1 else zero,
                                    zero if j == M - 1 else g,
                                    data_range, win_size, sigma, K)
        if gx is not None:  # the coarser level's gradient, spread back
            dlx = dlx + avg_pool2_adjoint(gx, *lx.shape[-2:])
            dly = dly + avg_pool2_adjoint(gy, *ly.shape[-2:])
        gx, gy = dlx, dly
    return gx, gy


def valid_correlate_adjoint(m: np.ndarray, k: np.ndarray, H: int, W: int) -> np.ndarray:
    """sum_p k(q - p) m(p): the adjoint of valid_correlate2d with the 2-D
    kernel k, from its (H-kh+1) x (W-kw+1) grid back onto H x W."""
    kh, kw = k.shape
    oh, ow = m.shape[-2:]
    out = np.zeros(m.shape[:-2] + (H, W), dtype=np.float64)
    for i in range(kh):
        for j in range(kw):
            out[..., i:i + oh, j:j + ow] += k[i, j] * m
    return out


def gms_stats_grad(x, y, data_range=255.0, T=None, downsample=True, eps=None,
                   g_mean=None, g_std=None) -> Tuple[np.ndarray, np.ndarray]:
    """d L / d x and d L / d y in float64 for
    L = sum_n g_mean[n] mean(q_n) + g_std[n] std(q_n), the per-image mean and
    population standard deviation of the GMS map over its channels (the
    statistics of gmsd_stats; reference functional.py:959-971).

    By the chain rule: dmean/dq = 1/n, dstd/dq = (q - m)/(n std);
    dq/dg1 = 2 (g2 D - g1 N)/D^2 with N = 2 g1 g2 + T, D = g1^2 + g2^2 + T;
    dg/dgx = gx/g, dg/dgy = gy/g; the Prewitt correlations' adjoints; and the
    2x2 mean's adjoint (a quarter to each pixel of the block, none to the
    dropped odd row / column)."""
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    N, C, H, W = x.shape
    L = float(data_range)
    T = 170.0 * (L / 255.0) ** 2 if T is None else float(T)
    eps = (1e-6 * L) ** 2 if eps is None else float(eps)
    gm = np.zeros(N) if g_mean is None else np.asarray(g_mean, np.float64)
    gs = np.zeros(N) if g_std is None else np.asarray(g_std, np.float64)
    xs, ys = (avg_pool2(x), avg_pool2(y)) if downsample else (x, y)
    Hd, Wd = xs.shape[-2:]
    gx1, gy1 = valid_correlate2d(xs, PREWITT_X), valid_correlate2d(xs, PREWITT_Y)
    gx2, gy2 = valid_correlate2d(ys, PREWITT_X), valid_correlate2d(ys, PREWITT_Y)
    g1 = np.sqrt(gx1 ** 2 + gy1 ** 2 + eps)
    g2 = np.sqrt(gx2 ** 2 + gy2 ** 2 + eps)
    num = 2.0 * g1 * g2 + T
    den = g1 * g1 + g2 * g2 + T
    q = num / den
    n = q[0].size
    flat = q.reshape(N, -1)
    m = flat.mean(axis=1)
    sd = np.sqrt(((flat - m[:, None]) ** 2).mean(axis=1))
    with np.errstate(divide="ignore", invalid="ignore"):
        ks = np.where(sd > 0, gs / (n * sd), 0.0)
    w = gm[:, None, None, None] / n + ks[:, None, None, None] * (q - m[:, None, None, None])
    d1 = w * 2.0 * (g2 * den - g1 * num) / den ** 2
    d2 = w * 2.0 * (g1 * den - g2 * num) / den ** 2
    dxs = (valid_correlate_adjoint(d1 * gx1 / g1, PREWITT_X, Hd, Wd)
           + valid_correlate_adjoint(d1 * gy1 / g1, PREWITT_Y, Hd, Wd))
    dys = (valid_correlate_adjoint(d2 * gx2 / g2, PREWITT_X, Hd, Wd)
           + valid_correlate_adjoint(d2 * gy2 / g2, PREWITT_Y, Hd, Wd))
    if not downsample:
        return dxs, dys

    def spread(ds):
        out = np.zeros((N, C, H, W))
        out[..., :2 * Hd, :2 * Wd] = 0.25 * np.repeat(np.repeat(ds, 2, axis=-2), 2, axis=-1)
        return out

    return spread(dxs), spread(dys)

