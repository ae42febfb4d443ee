// Shared device helpers for the gfx950 metric kernels.
//
// Everything here is written for CDNA4: 64-lane wavefronts, 256-thread
// workgroups (4 waves), full-rate FP64 vector arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "fa_abi.h"

namespace fa {

constexpr int WAVE = 64;
constexpr int BLOCK = 256;  // threads per workgroup for every kernel here
constexpr int WAVES_PER_BLOCK = BLOCK / WAVE;

// --------------------------------------------------------------------------
// element types
//
// The narrow float types travel as raw 16-bit patterns; bfloat16 widens by a
// shift and half through the hardware conversion.
// --------------------------------------------------------------------------
struct half_t { uint16_t bits; };
struct bf16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<uint8_t> {
  __device__ static inline float f(uint8_t v) { return static_cast<float>(v); }
  __device__ static inline double d(uint8_t v) { return static_cast<double>(v); }
};
template <> struct Elem<float> {
  __device__ static inline float f(float v) { return v; }
  __device__ static inline double d(float v) { return static_cast<double>(v); }
};
template <> struct Elem<double> {
  __device__ static inline float f(double v) { return static_cast<float>(v); }
  __device__ static inline double d(double v) { return v; }
};
template <> struct Elem<half_t> {
  __device__ static inline float f(half_t v) {
    __half_raw r;
    r.x = v.bits;
    return __half2float(__half(r));
  }
  __device__ static inline double d(half_t v) { return static_cast<double>(f(v)); }
};
template <> struct Elem<bf16_t> {
  __device__ static inline float f(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
  }
  __device__ static inline double d(bf16_t v) { return static_cast<double>(f(v)); }
};

// Load one element at working precision CT (float or double).
template <typename CT, typename T>
__device__ inline CT load_as(const T* p, int64_t i) {
  if constexpr (sizeof(CT) == 8) return Elem<T>::d(p[i]);
  else return Elem<T>::f(p[i]);
}

// --------------------------------------------------------------------------
// wave64 / workgroup reductions
//
// A butterfly over all 64 lanes, then one slot per wave in LDS; the result is
// valid in thread 0 only.  The order of additions is fixed, so every sum in
// this library is deterministic run to run.
// --------------------------------------------------------------------------
// Lane i receives lane i+1's value; lane 63 receives 0.  One DPP move across
// the whole wave (wave_shl:1, a VALU op) instead of the LDS round trip of
// ds_bpermute that __shfl_down takes.
__device__ inline int wave_next(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x130, 0xf, 0xf, true);
}
__device__ inline float wave_next(float v) {
  return __int_as_float(wave_next(__float_as_int(v)));
}
__device__ inline double wave_next(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = wave_next(static_cast<int>(b & 0xffffffff));
  const int hi = wave_next(static_cast<int>(b >> 32));
  return __longlong_as_double((static_cast<int64_t>(hi) << 32) |
                              static_cast<int64_t>(static_cast<uint32_t>(lo)));
}

// Lane i receives lane i ^ 1's value: DPP quad_perm:[1,0,3,2], a VALU op.
__device__ inline int lane_xor1(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);
}
__device__ inline float lane_xor1(float v) {
  return __int_as_float(lane_xor1(__float_as_int(v)));
}
__device__ inline double lane_xor1(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = lane_xor1(static_cast<int>(b & 0xffffffff));
  const int hi = lane_xor1(static_cast<int>(b >> 32));
  return __longlong_as_double((static_cast<int64_t>(hi) << 32) |
                              static_cast<int64_t>(static_cast<uint32_t>(lo)));
}

template <typename V>
__device__ inline V wave_sum(V v) {
#pragma unroll
  for (int off = WAVE / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}

template <typename V, int NT = BLOCK>
__device__ inline V block_sum(V v, V* smem /* >= NT / WAVE */) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  V out = V(0);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < NT / WAVE; ++i) out += smem[i];
  }
  return out;
}

// Two independent sums in one pass; smem holds 2 * WAVES_PER_BLOCK slots.
template <typename V>
__device__ inline void block_sum2(V a, V b, V* smem, V* oa, V* ob) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  if (lane == 0) {
    smem[wave] = a;
    smem[WAVES_PER_BLOCK + wave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    V sa = V(0), sb = V(0);
#pragma unroll
    for (int i = 0; i < WAVES_PER_BLOCK; ++i) {
      sa += smem[i];
      sb += smem[WAVES_PER_BLOCK + i];
    }
    *oa = sa;
    *ob = sb;
  }
}

// --------------------------------------------------------------------------
// XCD-aware tile order
//
// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs, each
// with a private L2.  Tiles that share input rows / columns (neighbouring
// strips and row chunks of one plane) should run on the same XCD, so tile t is
// given to workgroup (t % 8)-major: XCD x takes tiles [x*q, (x+1)*q) in order.
// The map is a bijection of [0, total) when total is a multiple of 8 and the
// identity otherwise.
// --------------------------------------------------------------------------
constexpr unsigned NUM_XCD = 8;

__device__ inline unsigned xcd_tile(unsigned wg, unsigned total) {
  if (total % NUM_XCD != 0) return wg;
  return (wg % NUM_XCD) * (total / NUM_XCD) + wg / NUM_XCD;
}

}  // namespace fa

// --------------------------------------------------------------------------
// host-side plumbing shared by the entry points
// --------------------------------------------------------------------------
#define FA_HIP_TRY(EXPR)                                                 \
  do {                                                                   \
    const hipError_t e_ = (EXPR);                                        \
    if (e_ != hipSuccess) return -static_cast<int>(e_);                  \
  } while (0)

#define FA_LAUNCH_CHECK()                                                \
  do {                                                                   \
    const hipError_t e_ = hipGetLastError();                             \
    if (e_ != hipSuccess) return -static_cast<int>(e_);                  \
  } while (0)

namespace fa {

// Makes `dev` current for the duration of one entry point and restores the
// caller's device afterwards (the caller's notion of "current" is torch's).
struct DeviceScope {
  int prev = -1;
  bool changed = false;
  hipError_t status = hipSuccess;
  explicit DeviceScope(int dev) {
    status = hipGetDevice(&prev);
    if (status == hipSuccess && dev >= 0 && dev != prev) {
      status = hipSetDevice(dev);
      changed = (status == hipSuccess);
    }
  }
  ~DeviceScope() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// Compute-unit count of `device`, cached: the attribute query costs as much
// as a small kernel.
int cu_count(int device);

// Launches the per-row / total mean reduction over a [nrows, ncols] array of
// 8-byte partials (uint64 when `exact`, float64 otherwise).  Skipped when every
// sink is null.  Defined in fa_pixel.hip.
int launch_finalize(const void* partial, bool exact, int nrows, int ncols,
                    double n_per_row, double n_total, double psnr_bias,
                    double* out_per_row, double* out_total,
                    double* out_psnr_per_row, double* out_psnr_total,
                    hipStream_t st);

// Stores a lane may or may not make, issued on every path: a buffer resource
// over one output row (scalar base, range: the row's bytes, or nothing for a
// null output) and the lane's byte offset in it, or 0x80000000 -- past every
// range -- where the lane has nothing to store, so the range check drops it.
template <typename E>
__device__ inline __amdgpu_buffer_rsrc_t row_rsrc(E* row, int ncols) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<typename std::remove_const<E>::type*>(row), 0,
                                           row ? ncols * static_cast<int>(sizeof(E)) : 0,
                                           0x00020000);
}
template <typename E>
__device__ inline uint32_t lane_off(int col, bool on) {
  return on ? static_cast<uint32_t>(col) * static_cast<uint32_t>(sizeof(E)) : 0x80000000u;
}
__device__ inline void row_store(float v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}
__device__ inline void row_store(double v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, off, 0, 0);
}

// --------------------------------------------------------------------------
// The one-launch finish of the SSIM forwards (fa_gpu_ssim_once: the uint8
// matrix-core kernel and the strip kernel).
//
// Each workgroup adds its sum of the SSIM map to its image's accumulator word
// as a signed fixed-point integer, round(sum * 2^F), packed with a
// contribution count: word = (value << SSIM_FIN_COUNT_BITS) + count, in two's
// complement (the count stays in the low bits whatever the sign of the sum,
// and an arithmetic shift recovers the sum).  One returning device-scope
// atomic adds both; integer addition does not depend on the order, so the
// result is the same from run to run.  The workgroup whose add completes an
// image's count (C * tiles workgroups) holds the image's sum, writes its mean,
// resets the word, and adds the image's integer sum to the batch word, counted
// in images, whose completer writes the batch mean.  F = 51 - bits(2 N pixels
// per image) keeps every packed sum within the word (SSIM values lie in
// [-1, 1] where C1, C2 > 0; the host takes the finish only then).  Words sit
// on their own 128-byte lines.
//
// Floating input can hold NaN or inf, which make SSIM values NaN, and a
// fixed-point word cannot: a workgroup whose sum is not finite adds 0 to the
// value and sets the word's flag, the next word of its line, with a returning
// atomic whose value it waits for before its count add; the completer then
// reads and clears the flag by an exchange and writes NaN, as the reference's
// float mean would be (and the batch's flag likewise).  A flag set before a
// count add is performed before it, so the completer, whose add saw every
// count, sees every flag.
// --------------------------------------------------------------------------
constexpr int SSIM_FIN_COUNT_BITS = 12;
constexpr int SSIM_FIN_STRIDE = 16;
constexpr int SSIM_FIN_MAX_IMAGES = 256;
static_assert(FA_SSIM_ACC_WORDS == (SSIM_FIN_MAX_IMAGES + 1) * SSIM_FIN_STRIDE,
              "the ABI's accumulator size");

struct SsimFin {
  uint64_t* acc;              // FA_SSIM_ACC_WORDS, zero; left zero
  double fscale, finv;        // 2^F and 2^-F
  double npix_img, npix_all;  // output pixels of one image, of the batch
  int N;
  double* out_per_image;
  double* out_total;
};

// The host's F for a batch of npix_all output pixels; false where too few
// fraction bits would be left (never at real sizes).
inline bool ssim_fin_scale(SsimFin& f) {
  int bits = 1;
  while (bits < 50 && static_cast<double>(int64_t(1) << bits) <= 2.0 * f.npix_all) ++bits;
  f.fscale = static_cast<double>(int64_t(1) << (51 - bits));
  f.finv = 1.0 / f.fscale;
  return bits < 40;
}

// The NaN flags of the one-launch finishes (SSIM here, GMSD in fa_gmsd.hip).
// fin_flag_set sets flag word `flag` and waits for the atomic's return, so
// that it is performed before anything the thread issues after it;
// fin_flag_take reads and clears it.
__device__ inline void fin_flag_set(uint64_t* flag) {
  const uint64_t r = __hip_atomic_fetch_or(flag, uint64_t(1), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(r));  // the value is used: what follows issues after it is back
}

__device__ inline bool fin_flag_take(uint64_t* flag) {
  return __hip_atomic_exchange(flag, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Thread-level: workgroup sum `s` of image `img`, whose words take
// `wg_per_image` contributions.
__device__ inline void ssim_fin_add(const SsimFin& f, int img, int wg_per_image, double s) {
  constexpr uint64_t CM = (uint64_t(1) << SSIM_FIN_COUNT_BITS) - 1;
  constexpr double NaN = __builtin_nan("");
  uint64_t* w = f.acc + static_cast<int64_t>(img) * SSIM_FIN_STRIDE;
  const bool finite = __builtin_isfinite(s);
  if (!finite) fin_flag_set(w + 1);
  const int64_t q = finite ? __double2ll_rn(s * f.fscale) : 0;
  const uint64_t old = __hip_atomic_fetch_add(
      w, (static_cast<uint64_t>(q) << SSIM_FIN_COUNT_BITS) + 1u, __ATOMIC_RELAXED,
      __HIP_MEMORY_SCOPE_AGENT);
  if ((old & CM) + 1u != static_cast<uint64_t>(wg_per_image)) return;
  __hip_atomic_store(w, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool nan_img = fin_flag_take(w + 1);
  const int64_t tot = (static_cast<int64_t>(old) >> SSIM_FIN_COUNT_BITS) + q;
  if (f.out_per_image)
    f.out_per_image[img] = nan_img ? NaN : static_cast<double>(tot) * f.finv / f.npix_img;
  if (!f.out_total) return;
  uint64_t* wb = f.acc + static_cast<int64_t>(SSIM_FIN_MAX_IMAGES) * SSIM_FIN_STRIDE;
  if (nan_img) fin_flag_set(wb + 1);
  const uint64_t ob = __hip_atomic_fetch_add(
      wb, (static_cast<uint64_t>(tot) << SSIM_FIN_COUNT_BITS) + 1u, __ATOMIC_RELAXED,
      __HIP_MEMORY_SCOPE_AGENT);
  if ((ob & CM) + 1u != static_cast<uint64_t>(f.N)) return;
  __hip_atomic_store(wb, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool nan_all = fin_flag_take(wb + 1);
  const int64_t all = (static_cast<int64_t>(ob) >> SSIM_FIN_COUNT_BITS) + tot;
  *f.out_total = nan_all ? NaN : static_cast<double>(all) * f.finv / f.npix_all;
}

}  // namespace fa

#define FA_DEVICE_SCOPE(DEV)                                             \
  fa::DeviceScope guard_(DEV);                                           \
  if (guard_.status != hipSuccess) return -static_cast<int>(guard_.status)
