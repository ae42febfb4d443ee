// The MS-SSIM pyramid step on gfx950: non-overlapping 2x2 mean of x and y in
// one launch, odd trailing row / column dropped (the avg_pool2d convention of
// reference functional.py:876-885 and reference.py:231-241).
//
// The output type is chosen so that the levels are exact: uint8 pools into
// float32 (a sum of four bytes needs 10 bits, the 1/4 scale is a power of two)
// and every floating input into float64 (exact for float16, and for float32 /
// bfloat16 whenever the four values of a block span less than 2^29 / 2^45 in
// magnitude; beyond that the mean is correctly rounded to 2^-53).  A pyramid
// this precise is what keeps the MS-SSIM gradient within 1e-6 of float64: the
// coarse scales amplify an input rounding of 6e-8 roughly a hundredfold.
//
// Each lane produces two adjacent output samples per tensor from a 2x4 input
// block, so a wave reads 2 x 256 consecutive input elements per row pair.
#include "fa_common.h"

namespace fa {

template <typename T, typename O>
__global__ __launch_bounds__(BLOCK) void pool2_kernel(const T* __restrict__ x,
                                                      const T* __restrict__ y, int H, int W,
                                                      int Hd, int Wd, int64_t total_pairs,
                                                      O* __restrict__ ox, O* __restrict__ oy) {
  const int pairs_per_row = (Wd + 1) / 2;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x; t < total_pairs;
       t += static_cast<int64_t>(gridDim.x) * BLOCK) {
    const int64_t row_id = t / pairs_per_row;          // (plane, output row)
    const int j0 = 2 * static_cast<int>(t - row_id * pairs_per_row);
    const int64_t plane = row_id / Hd;
    const int i = static_cast<int>(row_id - plane * Hd);
    const int64_t in0 = plane * H * W + static_cast<int64_t>(2 * i) * W;
    const int64_t out0 = plane * Hd * Wd + static_cast<int64_t>(i) * Wd;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int j = j0 + k;
      if (j < Wd) {
        const int64_t a = in0 + 2 * j;
        ox[out0 + j] = O(0.25) * (load_as<O>(x, a) + load_as<O>(x, a + 1) +
                                  load_as<O>(x, a + W) + load_as<O>(x, a + W + 1));
        oy[out0 + j] = O(0.25) * (load_as<O>(y, a) + load_as<O>(y, a + 1) +
                                  load_as<O>(y, a + W) + load_as<O>(y, a + W + 1));
      }
    }
  }
}

template <typename T, typename O>
static void launch_pool(hipStream_t st, const void* x, const void* y, int H, int W, int Hd,
                        int Wd, int64_t pairs, void* ox, void* oy, int cus) {
  const int64_t want = (pairs + BLOCK - 1) / BLOCK;
  const int64_t cap = static_cast<int64_t>(cus) * 16;
  const unsigned grid = static_cast<unsigned>(want < cap ? want : cap);
  hipLaunchKernelGGL((pool2_kernel<T, O>), dim3(grid), dim3(BLOCK), 0, st,
                     static_cast<const T*>(x), static_cast<const T*>(y), H, W, Hd, Wd, pairs,
                     static_cast<O*>(ox), static_cast<O*>(oy));
}

}  // namespace fa

using namespace fa;

extern "C" {

FA_API int fa_gpu_pool2(const void* x, const void* y, int dtype, int planes, int H, int W,
                        void* ox, void* oy, int out_dtype, int device, void* stream) {
  if (!x || !y || !ox || !oy) return FA_E_ARG;
  if (planes <= 0 || H < 2 || W < 2) return FA_E_SHAPE;
  if (dtype < FA_U8 || dtype > FA_F64) return FA_E_DTYPE;
  // the pyramid rule: uint8 to float32, every floating type to float64
  if (out_dtype != (dtype == FA_U8 ? FA_F32 : FA_F64)) return FA_E_DTYPE;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Hd = H / 2, Wd = W / 2;
  const int64_t pairs = static_cast<int64_t>(planes) * Hd * ((Wd + 1) / 2);
  const int cus = cu_count(device);
  switch (dtype) {
    case FA_U8: launch_pool<uint8_t, float>(st, x, y, H, W, Hd, Wd, pairs, ox, oy, cus); break;
    case FA_F16: launch_pool<half_t, double>(st, x, y, H, W, Hd, Wd, pairs, ox, oy, cus); break;
    case FA_BF16: launch_pool<bf16_t, double>(st, x, y, H, W, Hd, Wd, pairs, ox, oy, cus); break;
    case FA_F32: launch_pool<float, double>(st, x, y, H, W, Hd, Wd, pairs, ox, oy, cus); break;
    default: launch_pool<double, double>(st, x, y, H, W, Hd, Wd, pairs, ox, oy, cus); break;
  }
  FA_LAUNCH_CHECK();
  return FA_OK;
}

}  // extern "C"
