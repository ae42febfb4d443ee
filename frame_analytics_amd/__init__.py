"""frame_analytics_amd -- MSE / PSNR / SSIM / MS-SSIM / GMSD on AMD MI355X.

A drop-in for the fused metric kernels of NevermindNilas/frame_analytics:
the same ``fa.ssim / fa.ms_ssim / fa.psnr / fa.mse / fa.l1 / fa.gmsd`` API,
served on the GPU by hand-written gfx950 HIP kernels behind a C ABI
(``include/fa_abi.h``, ``libfa_gpu.so``).

Usage, scoring a batch of decoded frames against their sources::

    import frame_analytics_amd as fa
    # src, out: (N, 3, H, W) uint8 tensors on the GPU
    db = fa.psnr(src, out)                    # exact integer SSE, dB in-kernel
    s = fa.ssim(src, out, reduction="none")   # one value per frame
    loss = 1 - fa.ms_ssim(pred, target, data_range=1.0)  # float32, differentiable
"""

from .functional import (  # noqa: F401
    MS_SSIM_WEIGHTS,
    charbonnier,
    gaussian_window_1d,
    gms,
    gmsd,
    huber,
    l1,
    ms_ssim,
    mse,
    psnr,
    rgb_to_luma,
    set_compile_enabled,
    ssim,
)
from .modules import (  # noqa: F401
    GMSD,
    MSE,
    PSNR,
    SSIM,
    Charbonnier,
    Huber,
    L1,
    MSSSIM,
    StreamingMetrics,
)

__version__ = "0.1.0"

__all__ = [
    "mse", "psnr", "ssim", "ms_ssim", "gmsd", "gms", "l1", "charbonnier", "huber",
    "rgb_to_luma", "MSE", "PSNR", "SSIM", "MSSSIM", "GMSD", "L1", "Charbonnier",
    "Huber", "StreamingMetrics", "gaussian_window_1d", "set_compile_enabled",
    "backend_status", "MS_SSIM_WEIGHTS",
]


def backend_status() -> dict:
    """Whether the gfx950 kernel library is loaded, and why not if it is not."""
    from . import backend

    return backend.status()
