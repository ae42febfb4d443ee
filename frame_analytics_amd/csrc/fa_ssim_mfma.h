// SSIM forward over uint8 planes on the matrix cores (fa_ssim_mfma.hip).
#pragma once

#include "fa_common.h"

namespace fa {

// One fa_gpu_ssim(_ex) / fa_gpu_ssim_cs(_ex) call over uint8 planes without
// luma, or (CS pass only) over the planes of a uint8 input's 2 x 2 pyramid.
struct SsimMfmaCall {
  enum Src {
    U8 = 0,         // uint8 samples
    F32_LEVEL = 1,  // float32 samples, multiples of 4^-s in [0, 255], s <= 4
    F16_LEVEL = 2,  // float16 samples, multiples of 1/4 in [0, 255] (level 1)
  };
  const void* x;
  const void* y;
  int src;                     // Src
  int64_t xsn, xsc, ysn, ysc;  // image and channel strides (elements)
  int xsh, ysh;                // row strides
  int N, C, H, W, Hout, Wout, K;
  const float* win;            // the 1-D window, K floats on the device
  double C1, C2;
  float* map;                  // optional float32 SSIM map (N, C, Hout, Wout)
  double* partial;             // per-plane partial sums, bpp slots per plane
  int bpp;
  // MS-SSIM's CS pass (partial_cs non-null): per-plane sums of SSIM (unless
  // partial is null) and of cs = A2 / B2, and optionally the next pyramid
  // level, the 2 x 2 means of x
  // and y (floor(H/2) x floor(W/2) per plane) into px / py: float32, or
  // float16 when level_f16 (uint8 input only: quarter samples are exact)
  double* partial_cs;
  void* px;
  void* py;
  bool level_f16;
  // the one-launch finish (forward over uint8 planes, no map): a zeroed
  // accumulator of FA_SSIM_ACC_WORDS words the launch leaves zeroed, and the
  // outputs it then writes itself (either may be null, not both)
  uint64_t* acc;
  double* out_per_image;
  double* out_total;
};

// Launches the matrix-core SSIM forward (or CS pass) when the call fits it
// (rows and planes aligned to 8 samples, 8-byte (uint8) or 16-byte (levels)
// aligned bases, K <= 16, enough partial slots, 16-byte aligned pyramid
// output planes).  Returns FA_OK and
// sets *tiles (partial slots used per plane) when it launched; returns FA_OK
// with *tiles = 0 when the call does not fit, so the caller runs the
// vector-ALU strip kernel instead.  With c.acc set, a launch that finished
// the call itself (no finalize needed) sets *tiles = -1.
int ssim_mfma(const SsimMfmaCall& c, int device, hipStream_t st, int* tiles);

// Inference MS-SSIM over uint8 planes without luma, M (3 .. 5) scales, in
// three launches: scale 0 (writing the float16 level 1), scale 1 (writing the
// float32 levels 2, 3 and 4), and scales 2 .. M - 1 side by side in one
// launch whose last workgroup also finishes the reduction from the
// per-(scale, plane) fixed-point sums every launch adds to `words`.
struct SsimMfmaMs {
  const void* x;
  const void* y;
  int64_t xsn, xsc, ysn, ysc;  // image and channel strides of the input (elements)
  int xsh, ysh;                // row strides
  int N, C, H, W, K, M;
  const float* win;            // the 1-D window, K floats on the device
  double C1, C2;
  const double* weights;       // host, M exponents
  void* lx[8];                 // level i >= 1 of x and y: floor(H / 2^i) x
  void* ly[8];                 //   floor(W / 2^i) per plane, float16 (i = 1), float32
  uint64_t* words;             // FA_MS_SSIM_ACC_WORDS, zero; left zero
  double* out_per_image;
  double* out_total;
};

// Launches it when every scale fits (ssim_mfma's layout rules at each scale,
// N * C <= 256, C1 and C2 positive) and sets *done; otherwise launches nothing
// and leaves *done false, for the per-scale path.
int ssim_mfma_ms(const SsimMfmaMs& c, int device, hipStream_t st, bool* done);

}  // namespace fa
