// GMSD / GMS on gfx950: optional 2x2 mean downsample, 3x3 Prewitt pair (taps
// +-1/3, 'valid' support), gradient-magnitude similarity
//     g = sqrt(gx^2 + gy^2 + eps),  q = (2 g1 g2 + T) / (g1^2 + g2^2 + T)
// and the per-image mean and population standard deviation of q
// (reference: fa_cuda.cu:926-1026, 1416-1466; reference.py:288-335).
//
// Layout on CDNA4: every wave owns a strip of 64 downsampled columns (62
// outputs, the last two lanes are the Prewitt halo) and walks down it with a
// three-row window in registers.  The column sums and row differences of the
// Prewitt pair need the two lanes to the right, which come from in-wave
// shuffles -- no LDS staging and no barriers.  For uint8 input the downsampled
// samples, their 3-sums and differences are all exact in float32, so they stay
// float32; every other input type carries them in float64.  From the Prewitt
// differences on, g and q are formed in float64 (full rate on CDNA4,
// and the kernel is bound on HBM), so q carries no float32 rounding into the
// standard deviation.  Sum q and sum q^2 are accumulated in float64 and reduced
// in a fixed order.
#include "fa_common.h"

#include <type_traits>

namespace fa {

constexpr int G_OUTW = WAVE - 2;                     // output columns per wave
constexpr int G_STRIP = WAVES_PER_BLOCK * G_OUTW;    // output columns per workgroup
constexpr int G_TH = 64;                             // output rows per workgroup

// Sample type: float32 is exact for uint8 (multiples of 1/4 below 1024),
// float64 for everything else.
template <typename T>
using GSample = typename std::conditional<std::is_same<T, uint8_t>::value, float, double>::type;

template <typename T, bool DOWN>
__device__ inline GSample<T> gmsd_sample(const T* __restrict__ p, int64_t plane_off, int W,
                                         int r, int c) {
  using S = GSample<T>;
  if constexpr (DOWN) {
    const int64_t o = plane_off + static_cast<int64_t>(2 * r) * W + 2 * c;
    return S(0.25) * (load_as<S>(p, o) + load_as<S>(p, o + 1) + load_as<S>(p, o + W) +
                      load_as<S>(p, o + W + 1));
  } else {
    return load_as<S>(p, plane_off + static_cast<int64_t>(r) * W + c);
  }
}

// Gradient magnitude at this lane's column from the three rows v0 (top),
// v1, v2 (bottom); lanes 62 and 63 produce garbage that is never used.
template <typename S>
__device__ inline double prewitt_mag(S v0, S v1, S v2, double eps) {
  const S cs = v0 + v1 + v2;  // column sum     (for gx)
  const S rd = v0 - v2;       // row difference (for gy)
  const S cs2 = __shfl_down(cs, 2, WAVE);
  const S rd1 = __shfl_down(rd, 1, WAVE);
  const S rd2 = __shfl_down(rd, 2, WAVE);
  const double gx = static_cast<double>(cs - cs2) / 3.0;
  const double gy = (static_cast<double>(rd) + static_cast<double>(rd1) +
                     static_cast<double>(rd2)) / 3.0;
  return sqrt(fma(gx, gx, fma(gy, gy, eps)));
}

template <typename T, bool DOWN>
__global__ __launch_bounds__(BLOCK) void gmsd_kernel(
    const T* __restrict__ x, const T* __restrict__ y, int H, int W, int Hd, int Wd,
    int Hout, int Wout, double Tc, double eps, int strips, int bpp,
    double* __restrict__ psum, double* __restrict__ psumsq) {
  __shared__ double sred[2 * WAVES_PER_BLOCK];
  const int t = static_cast<int>(xcd_tile(blockIdx.x, gridDim.x));
  const int plane = t / bpp;
  const int tile = t - plane * bpp;
  const int chunk = tile / strips;
  const int strip = tile - chunk * strips;
  const int wave = threadIdx.x / WAVE;
  const int lane = threadIdx.x % WAVE;
  const int col = strip * G_STRIP + wave * G_OUTW + lane;  // downsampled column
  const bool col_in = col < Wd;
  const bool col_out = lane < G_OUTW && col < Wout;
  const int r0 = chunk * G_TH;
  const int rows = min(G_TH, Hout - r0);
  const int64_t plane_off = static_cast<int64_t>(plane) * H * W;

  using S = GSample<T>;
  auto fetch = [&](int r, S& xv, S& yv) {
    if (col_in && r < Hd) {
      xv = gmsd_sample<T, DOWN>(x, plane_off, W, r, col);
      yv = gmsd_sample<T, DOWN>(y, plane_off, W, r, col);
    } else {
      xv = S(0);
      yv = S(0);
    }
  };

  S x0, x1, x2, y0, y1, y2, nx, ny;
  fetch(r0, x0, y0);
  fetch(r0 + 1, x1, y1);
  fetch(r0 + 2, nx, ny);
  double acc = 0.0, acc2 = 0.0;
  for (int o = 0; o < rows; ++o) {
    x2 = nx;
    y2 = ny;
    if (o + 1 < rows) fetch(r0 + o + 3, nx, ny);
    const double g1 = prewitt_mag(x0, x1, x2, eps);
    const double g2 = prewitt_mag(y0, y1, y2, eps);
    const double q = (2.0 * g1 * g2 + Tc) / (g1 * g1 + g2 * g2 + Tc);
    if (col_out) {
      acc += q;
      acc2 += q * q;
    }
    x0 = x1;
    x1 = x2;
    y0 = y1;
    y1 = y2;
  }
  double s = 0.0, s2 = 0.0;
  block_sum2(acc, acc2, sred, &s, &s2);
  if (threadIdx.x == 0) {
    const int64_t o = static_cast<int64_t>(plane) * bpp + tile;
    psum[o] = s;
    psumsq[o] = s2;
  }
}

// Block b reduces image b: mean and population standard deviation of its map
// (reference fa_cuda.cu:1005-1026).
__global__ __launch_bounds__(BLOCK) void gmsd_finalize_kernel(
    const double* __restrict__ psum, const double* __restrict__ psumsq, int ncols,
    double npix, double* __restrict__ out_mean, double* __restrict__ out_std) {
  __shared__ double smem[2 * WAVES_PER_BLOCK];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * ncols;
  double a = 0.0, b = 0.0;
  for (int i = threadIdx.x; i < ncols; i += BLOCK) {
    a += psum[base + i];
    b += psumsq[base + i];
  }
  double sa = 0.0, sb = 0.0;
  block_sum2(a, b, smem, &sa, &sb);
  if (threadIdx.x == 0) {
    const double m = sa / npix;
    const double var = sb / npix - m * m;
    out_mean[blockIdx.x] = m;
    out_std[blockIdx.x] = sqrt(var > 0.0 ? var : 0.0);
  }
}

static int gmsd_geometry(int H, int W, int downsample, int* Hd, int* Wd, int* Hout,
                         int* Wout, int* strips, int* chunks) {
  if (H <= 0 || W <= 0) return FA_E_SHAPE;
  *Hd = downsample ? H / 2 : H;
  *Wd = downsample ? W / 2 : W;
  *Hout = *Hd - 2;
  *Wout = *Wd - 2;
  if (*Hout <= 0 || *Wout <= 0) return FA_E_SHAPE;
  *strips = (*Wout + G_STRIP - 1) / G_STRIP;
  *chunks = (*Hout + G_TH - 1) / G_TH;
  return FA_OK;
}

template <typename T>
static void launch_gmsd_t(bool down, dim3 grid, hipStream_t st, const void* x,
                          const void* y, int H, int W, int Hd, int Wd, int Hout,
                          int Wout, double Tc, double eps, int strips, int bpp,
                          double* psum, double* psumsq) {
  const T* tx = static_cast<const T*>(x);
  const T* ty = static_cast<const T*>(y);
  if (down)
    hipLaunchKernelGGL((gmsd_kernel<T, true>), grid, dim3(BLOCK), 0, st, tx, ty, H, W, Hd, Wd,
                       Hout, Wout, Tc, eps, strips, bpp, psum, psumsq);
  else
    hipLaunchKernelGGL((gmsd_kernel<T, false>), grid, dim3(BLOCK), 0, st, tx, ty, H, W, Hd, Wd,
                       Hout, Wout, Tc, eps, strips, bpp, psum, psumsq);
}

}  // namespace fa

using namespace fa;

extern "C" {

// reference: fa_cuda.cu:1416-1424 (fa_cuda_gmsd_workspace)
FA_API int fa_gpu_gmsd_workspace(int H, int W, int downsample, int* out_bpp) {
  if (!out_bpp) return FA_E_ARG;
  int Hd, Wd, Hout, Wout, strips, chunks;
  const int rc = gmsd_geometry(H, W, downsample, &Hd, &Wd, &Hout, &Wout, &strips, &chunks);
  if (rc != FA_OK) return rc;
  *out_bpp = strips * chunks;
  return FA_OK;
}

// reference: fa_cuda.cu:1426-1466 (fa_cuda_gmsd)
FA_API int fa_gpu_gmsd(const void* x, const void* y, int dtype, int N, int C,
                       int H, int W, double Tc, double eps, int downsample,
                       double* psum, double* psumsq, int bpp, double* out_mean,
                       double* out_std, int device, void* stream) {
  if (!x || !y || !psum || !psumsq || !out_mean || !out_std) return FA_E_ARG;
  if (N <= 0 || C <= 0) return FA_E_SHAPE;
  int Hd, Wd, Hout, Wout, strips, chunks;
  const int rc = gmsd_geometry(H, W, downsample, &Hd, &Wd, &Hout, &Wout, &strips, &chunks);
  if (rc != FA_OK) return rc;
  if (bpp != strips * chunks) return FA_E_ARG;
  const int64_t total = static_cast<int64_t>(N) * C * bpp;
  if (total > static_cast<int64_t>(INT32_MAX) / BLOCK) return FA_E_SHAPE;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(total));
  const bool down = downsample != 0;
  const double T = Tc, e = eps;
  switch (dtype) {
    case FA_U8: launch_gmsd_t<uint8_t>(down, grid, st, x, y, H, W, Hd, Wd, Hout, Wout, T, e, strips, bpp, psum, psumsq); break;
    case FA_F16: launch_gmsd_t<half_t>(down, grid, st, x, y, H, W, Hd, Wd, Hout, Wout, T, e, strips, bpp, psum, psumsq); break;
    case FA_BF16: launch_gmsd_t<bf16_t>(down, grid, st, x, y, H, W, Hd, Wd, Hout, Wout, T, e, strips, bpp, psum, psumsq); break;
    case FA_F32: launch_gmsd_t<float>(down, grid, st, x, y, H, W, Hd, Wd, Hout, Wout, T, e, strips, bpp, psum, psumsq); break;
    case FA_F64: launch_gmsd_t<double>(down, grid, st, x, y, H, W, Hd, Wd, Hout, Wout, T, e, strips, bpp, psum, psumsq); break;
    default: return FA_E_DTYPE;
  }
  FA_LAUNCH_CHECK();
  hipLaunchKernelGGL(gmsd_finalize_kernel, dim3(static_cast<unsigned>(N)), dim3(BLOCK), 0, st,
                     psum, psumsq, C * bpp, static_cast<double>(Hout) * Wout * C, out_mean,
                     out_std);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

}  // extern "C"
