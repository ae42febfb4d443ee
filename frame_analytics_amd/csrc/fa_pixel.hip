// Pixel losses on gfx950: MSE / L1 / Charbonnier / Huber, and PSNR folded
// into the final reduction.
//
// Behaviour follows the reference's pixel_kernel_u8 / pixel_kernel /
// finalize_kernel (reference: fa_cuda.cu:182-210, 252-359, 1065-1156):
// per-image sums, divided (never multiplied by a reciprocal) by the element
// count, optionally turned into dB as psnr_bias - 10*log10(mse).
//
// The design is CDNA4's own:
//   * large contiguous batches (>= 4 Mi elements per image) take the sweep:
//     one workgroup per CU walks the whole batch as one flat run of 16-byte
//     vectors (global_load_dwordx4), so the grid reads a compact window of
//     each tensor at any moment, and each wave follows the image edges
//     itself (pix_sweep_kernel).  Smaller or misaligned batches take a
//     (bpi, N) grid with four vectors in flight per lane per tensor.
//   * the exact uint8 sums never leave the integer pipe: squared error is
//     sum(a^2) + sum(b^2) - 2*sum(ab), three v_dot4_u32_u8 per dword pair, and
//     absolute error is one v_sad_u8 per dword pair.  Lane sums are flushed to
//     uint64 every unrolled step and the workgroup partials stay uint64, so the
//     batch total is exact for any element count.
//   * a pair of views whose misalignment differs is not pushed to a scalar
//     kernel: the widest vector width both share (16, 4 or 1 bytes) is used,
//     and each image peels its own unaligned head.
//   * float inputs compute the MSE / L1 / Huber term in float64 (full rate on
//     CDNA4); Charbonnier keeps a float32 square root unless the input is
//     float64, like the reference.
#include "fa_common.h"

#include <algorithm>
#include <type_traits>

namespace fa {

#ifndef FA_PIX_UNROLL
#define FA_PIX_UNROLL 4
#endif
#ifndef FA_PIX_WG_PER_CU
#define FA_PIX_WG_PER_CU 8
#endif
constexpr int PIX_UNROLL = FA_PIX_UNROLL;  // independent vector loads in flight per tensor

// Streaming loads.  Every byte is read once, so the loads are non-temporal
// (measured on MI355X: a pure 16-byte read stream reaches ~6.7 TB/s this way
// against ~5.6 TB/s with default cache policy).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline uint32_t ld_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }
constexpr int PIX_WG_PER_CU = FA_PIX_WG_PER_CU;  // workgroups per CU the grid aims for
constexpr int PIX_MIN_ELEMS_PER_THREAD = 64;
// Images of at least this many elements get the sweep's workspace (bpi = one
// partial per wave of one workgroup per CU).  At 4 Mi elements one round of
// the sweep (2 strides of 256 x 512 vectors on a 256-CU part) spans no more
// than one image for every element size, which the sweep requires.
constexpr int64_t PIX_SWEEP_MIN_ELEMS = int64_t(1) << 22;

// The four penalties (reference fa_cuda.cu:252-260).  Huber in the branchless
// form 0.5*min(a,d)^2 + d*(a - min(a,d)), equal to torch's HuberLoss term.
template <int OP, typename A>
__device__ inline A pix_term(A d, A p) {
  if constexpr (OP == FA_OP_MSE) {
    return d * d;
  } else if constexpr (OP == FA_OP_L1) {
    return d < A(0) ? -d : d;
  } else if constexpr (OP == FA_OP_CHARB) {
    return sqrt(d * d + p);
  } else {
    const A a = d < A(0) ? -d : d;
    const A lo = a < p ? a : p;
    return A(0.5) * lo * lo + p * (a - lo);
  }
}

// --------------------------------------------------------------------------
// uint8
// --------------------------------------------------------------------------

// Lane accumulator for uint8 pairs.  MSE keeps sum(a^2)+sum(b^2) in `s` and
// sum(ab) in `t`; L1 keeps the SAD in `s`; the float ops keep `f`.
template <int OP>
struct U8Lane {
  uint32_t s = 0, t = 0;
  float f = 0.0f;
  uint64_t exact = 0;
  double wide = 0.0;

  __device__ inline void dword(uint32_t x, uint32_t y, float p) {
    if constexpr (OP == FA_OP_MSE) {
      s = __builtin_amdgcn_udot4(x, x, s, false);
      s = __builtin_amdgcn_udot4(y, y, s, false);
      t = __builtin_amdgcn_udot4(x, y, t, false);
    } else if constexpr (OP == FA_OP_L1) {
      s = __builtin_amdgcn_sad_u8(x, y, s);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float d = static_cast<float>((x >> (8 * k)) & 0xffu) -
                        static_cast<float>((y >> (8 * k)) & 0xffu);
        f += pix_term<OP, float>(d, p);
      }
    }
  }
  // Called at most every PIX_UNROLL*4 dwords: s <= 64 * 520200 < 2^32.
  __device__ inline void flush() {
    if constexpr (OP == FA_OP_MSE) {
      exact += static_cast<uint64_t>(s - 2u * t);
      s = 0;
      t = 0;
    } else if constexpr (OP == FA_OP_L1) {
      exact += static_cast<uint64_t>(s);
      s = 0;
    } else {
      wide += static_cast<double>(f);
      f = 0.0f;
    }
  }
  __device__ inline void byte(uint8_t x, uint8_t y, float p) {
    const int d = static_cast<int>(x) - static_cast<int>(y);
    if constexpr (OP == FA_OP_MSE) {
      exact += static_cast<uint64_t>(d * d);
    } else if constexpr (OP == FA_OP_L1) {
      exact += static_cast<uint64_t>(d < 0 ? -d : d);
    } else {
      wide += static_cast<double>(pix_term<OP, float>(static_cast<float>(d), p));
    }
  }
};

template <int OP, int V>
__global__ __launch_bounds__(BLOCK) void pix_u8_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, int64_t per,
    int bpi, float param, void* __restrict__ partial) {
  constexpr bool EXACT = (OP == FA_OP_MSE || OP == FA_OP_L1);
  __shared__ uint64_t s_u[WAVES_PER_BLOCK];
  __shared__ double s_d[WAVES_PER_BLOCK];

  const int img = blockIdx.y;
  const uint8_t* pa = a + static_cast<int64_t>(img) * per;
  const uint8_t* pb = b + static_cast<int64_t>(img) * per;
  // a and b share their misalignment modulo V (checked by the host), so one
  // head length aligns both.
  int64_t head = 0;
  if constexpr (V > 1) {
    head = static_cast<int64_t>((V - (reinterpret_cast<uintptr_t>(pa) & (V - 1))) & (V - 1));
    if (head > per) head = per;
  }
  // V == 1 has no vector body: the byte loop below covers the whole image
  const int64_t nvec = V > 1 ? (per - head) / V : 0;
  const int64_t body_end = head + nvec * V;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x;
  const int64_t gstride = static_cast<int64_t>(bpi) * BLOCK;

  U8Lane<OP> acc;
  if constexpr (V == 16) {
    const uint4* va = reinterpret_cast<const uint4*>(pa + head);
    const uint4* vb = reinterpret_cast<const uint4*>(pb + head);
    int64_t v = gtid;
    for (; v + (PIX_UNROLL - 1) * gstride < nvec; v += PIX_UNROLL * gstride) {
      uint4 xa[PIX_UNROLL], xb[PIX_UNROLL];
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) {
        xa[u] = ld_stream(va + v + u * gstride);
        xb[u] = ld_stream(vb + v + u * gstride);
      }
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) {
        acc.dword(xa[u].x, xb[u].x, param);
        acc.dword(xa[u].y, xb[u].y, param);
        acc.dword(xa[u].z, xb[u].z, param);
        acc.dword(xa[u].w, xb[u].w, param);
      }
      acc.flush();
    }
    for (; v < nvec; v += gstride) {
      const uint4 xa = ld_stream(va + v);
      const uint4 xb = ld_stream(vb + v);
      acc.dword(xa.x, xb.x, param);
      acc.dword(xa.y, xb.y, param);
      acc.dword(xa.z, xb.z, param);
      acc.dword(xa.w, xb.w, param);
      acc.flush();
    }
  } else if constexpr (V == 4) {
    const uint32_t* va = reinterpret_cast<const uint32_t*>(pa + head);
    const uint32_t* vb = reinterpret_cast<const uint32_t*>(pb + head);
    int64_t v = gtid;
    for (; v + (PIX_UNROLL - 1) * gstride < nvec; v += PIX_UNROLL * gstride) {
      uint32_t xa[PIX_UNROLL], xb[PIX_UNROLL];
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) {
        xa[u] = ld_stream(va + v + u * gstride);
        xb[u] = ld_stream(vb + v + u * gstride);
      }
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) acc.dword(xa[u], xb[u], param);
      acc.flush();
    }
    for (; v < nvec; v += gstride) {
      acc.dword(ld_stream(va + v), ld_stream(vb + v), param);
      acc.flush();
    }
  }
  // unaligned head and ragged tail of this image (the whole image when V == 1)
  for (int64_t i = gtid; i < head; i += gstride) acc.byte(pa[i], pb[i], param);
  for (int64_t i = body_end + gtid; i < per; i += gstride) acc.byte(pa[i], pb[i], param);

  const int64_t slot = static_cast<int64_t>(img) * bpi + blockIdx.x;
  if constexpr (EXACT) {
    const uint64_t s = block_sum(acc.exact, s_u);
    if (threadIdx.x == 0) reinterpret_cast<uint64_t*>(partial)[slot] = s;
  } else {
    const double s = block_sum(acc.wide, s_d);
    if (threadIdx.x == 0) reinterpret_cast<double*>(partial)[slot] = s;
  }
}

// --------------------------------------------------------------------------
// float16 / bfloat16 / float32 / float64
// --------------------------------------------------------------------------
template <typename T, int OP, bool VEC>
__global__ __launch_bounds__(BLOCK) void pix_float_kernel(
    const T* __restrict__ a, const T* __restrict__ b, int64_t per, int bpi,
    double param, double* __restrict__ partial) {
  // Charbonnier's square root stays float32 unless the caller handed float64
  // (reference fa_cuda.cu:262-277); every other term is formed in float64.
  constexpr bool WIDE = (OP != FA_OP_CHARB) || sizeof(T) == 8;
  using A = typename std::conditional<WIDE, double, float>::type;
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  __shared__ double s_d[WAVES_PER_BLOCK];

  const int img = blockIdx.y;
  const T* pa = a + static_cast<int64_t>(img) * per;
  const T* pb = b + static_cast<int64_t>(img) * per;
  int64_t head = 0, nvec = 0;
  if constexpr (VEC) {
    head = static_cast<int64_t>((16 - (reinterpret_cast<uintptr_t>(pa) & 15)) & 15) /
           static_cast<int64_t>(sizeof(T));
    if (head > per) head = per;
    nvec = (per - head) / E;
  }
  const int64_t body_end = head + nvec * E;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x;
  const int64_t gstride = static_cast<int64_t>(bpi) * BLOCK;
  const A p = static_cast<A>(param);

  double acc = 0.0;
  if constexpr (VEC) {
    const uint4* va = reinterpret_cast<const uint4*>(pa + head);
    const uint4* vb = reinterpret_cast<const uint4*>(pb + head);
    int64_t v = gtid;
    for (; v + (PIX_UNROLL - 1) * gstride < nvec; v += PIX_UNROLL * gstride) {
      uint4 ra[PIX_UNROLL], rb[PIX_UNROLL];
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) {
        ra[u] = ld_stream(va + v + u * gstride);
        rb[u] = ld_stream(vb + v + u * gstride);
      }
      A part = A(0);
#pragma unroll
      for (int u = 0; u < PIX_UNROLL; ++u) {
        T ea[E], eb[E];
        __builtin_memcpy(ea, &ra[u], 16);
        __builtin_memcpy(eb, &rb[u], 16);
#pragma unroll
        for (int k = 0; k < E; ++k) {
          const A d = static_cast<A>(load_as<A>(ea, k)) - static_cast<A>(load_as<A>(eb, k));
          part += pix_term<OP, A>(d, p);
        }
      }
      acc += static_cast<double>(part);
    }
    for (; v < nvec; v += gstride) {
      const uint4 ra = ld_stream(va + v);
      const uint4 rb = ld_stream(vb + v);
      T ea[E], eb[E];
      __builtin_memcpy(ea, &ra, 16);
      __builtin_memcpy(eb, &rb, 16);
      A part = A(0);
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const A d = load_as<A>(ea, k) - load_as<A>(eb, k);
        part += pix_term<OP, A>(d, p);
      }
      acc += static_cast<double>(part);
    }
  }
  for (int64_t i = gtid; i < head; i += gstride) {
    const A d = load_as<A>(pa, i) - load_as<A>(pb, i);
    acc += static_cast<double>(pix_term<OP, A>(d, p));
  }
  for (int64_t i = body_end + gtid; i < per; i += gstride) {
    const A d = load_as<A>(pa, i) - load_as<A>(pb, i);
    acc += static_cast<double>(pix_term<OP, A>(d, p));
  }
  const double s = block_sum(acc, s_d);
  if (threadIdx.x == 0) partial[static_cast<int64_t>(img) * bpi + blockIdx.x] = s;
}

// --------------------------------------------------------------------------
// Large contiguous images: the sweep.
//
// One workgroup per CU, and the whole grid walks the batch as one flat run
// of 16-byte vectors: round r reads U gridwide strides of G*BLOCK
// consecutive vectors from each tensor, so at any moment the workgroups read
// a compact window of a few MB.  HBM3E serves that with better row locality
// than a (bpi, N) grid whose workgroups stream every image at once (measured
// on MI355X: configs[2] 55.4 us against 58.8 us per launch, 89.8% against
// 84.6% of 8 TB/s; 8 x 3 x 1080 x 1920 uint8 15.7 against 16.1 us).
//
// Images are contiguous, so a wave's vectors move from image to image as the
// run goes on.  Each wave tracks the image it is in (uniform) and the vector
// where the next one starts.  A round that lies wholly inside the image is a
// plain unpredicated burst of loads; only the about one round per image that
// reaches the edge (a round spans at most U*G*BLOCK <= nv vectors, checked by
// the host, so it touches at most two images) sorts its lanes into two
// accumulators.  Once every lane has passed the edge the wave sets its sum
// for that image aside in LDS, and after the walk each workgroup writes one
// partial per image (batches of more than SWEEP_LDS_IMAGES images write one
// per wave instead).  No barrier inside the walk: a workgroup partial formed
// behind a barrier at every image edge measured 3 us slower per launch, and a
// form that predicated every load ran at 74 us (at one or two waves per SIMD
// each extra instruction in a round is time with no load in flight).
// A single-launch form whose last workgroup also finalized (a counter that
// the caller zeroes once) measured no faster as a whole call: the finalize
// launch already overlaps the tail of the sweep.
// --------------------------------------------------------------------------
// Launch shape, from a sweep on MI355X (uint8 MSE kernel time; one workgroup
// per CU unless noted):
//   U x threads      4Kx8   1080p RGB x8   1080p RGB x32
//   4 x 256           55.7-56.1 us        16.8-17.2 us   58.3-58.6 us
//   2 x 512           55.7                15.9-16.2      56.5-58.8
//   2 x 256, 2/CU     56.6-56.7           16.0-16.4      56.4
//   1 x 1024          57.6                15.8-15.9      58.6
//   3 x 256           59.5-59.7           18.6-18.7      65.4-65.6
// Two waves per SIMD with two strides in flight each keep the same bytes in
// flight as one wave with four, but one wave's loads are issued while the
// other sums.
#ifndef FA_SWEEP_UNROLL
#define FA_SWEEP_UNROLL 2
#endif
#ifndef FA_SWEEP_BLOCK
#define FA_SWEEP_BLOCK 512
#endif
constexpr int SWEEP_UNROLL = FA_SWEEP_UNROLL;  // gridwide strides per round
constexpr int SWEEP_BLOCK = FA_SWEEP_BLOCK;    // threads per workgroup (one per CU)
constexpr int SWEEP_LDS_IMAGES = 32;           // batches up to this size sum waves in LDS
// uint8 batches below this many bytes per tensor take the many-wave shape: 16
// waves per CU with one 16-byte load in flight each per tensor, against 8
// waves with two (the same bytes in flight, the same round).  Measured per
// fa_gpu_pixel_reduce call, 8 / 16 / 24 x 3 x 1080 x 1920 and 5 / 6 / 7 x 3 x
// 2160 x 3840: 8-15 % faster; 8 / 9 / 12 / 16 x 3 x 2160 x 3840 (199 MB and up
// per tensor): 1.5-2.6 % slower, so those keep the two-load shape.
constexpr int64_t SWEEP_MANY_WAVES_BELOW = 190000000;
constexpr int SWEEP_MANY_BLOCK = 1024;
constexpr int SWEEP_SLOTS_PER_CU = SWEEP_MANY_BLOCK / WAVE;  // workspace: the larger shape

template <typename T, int OP>
struct VecAcc {
  static constexpr bool U8 = std::is_same<T, uint8_t>::value;
  static constexpr bool EXACT = U8 && (OP == FA_OP_MSE || OP == FA_OP_L1);
  static constexpr bool WIDE = (OP != FA_OP_CHARB) || sizeof(T) == 8;
  static constexpr int E = 16 / static_cast<int>(sizeof(T));
  using A = typename std::conditional<WIDE, double, float>::type;

  U8Lane<OP> u8;        // uint8
  A part = A(0);        // float types: this round
  double acc = 0.0;     // float types: flushed rounds

  __device__ inline void add(const uint4& ra, const uint4& rb, float p8, A p) {
    if constexpr (U8) {
      u8.dword(ra.x, rb.x, p8);
      u8.dword(ra.y, rb.y, p8);
      u8.dword(ra.z, rb.z, p8);
      u8.dword(ra.w, rb.w, p8);
    } else {
      T ea[E], eb[E];
      __builtin_memcpy(ea, &ra, 16);
      __builtin_memcpy(eb, &rb, 16);
#pragma unroll
      for (int k = 0; k < E; ++k) part += pix_term<OP, A>(load_as<A>(ea, k) - load_as<A>(eb, k), p);
    }
  }
  // The vector's terms go to this accumulator, or to `other` where `hi` is
  // set: lane-wise selects, no divergent branch.
  __device__ inline void add_split(const uint4& ra, const uint4& rb, float p8, A p, bool hi,
                                   VecAcc& other) {
    VecAcc t;
    t.add(ra, rb, p8, p);
    if constexpr (U8) {
      u8.s += hi ? 0u : t.u8.s;
      other.u8.s += hi ? t.u8.s : 0u;
      if constexpr (OP == FA_OP_MSE) {
        u8.t += hi ? 0u : t.u8.t;
        other.u8.t += hi ? t.u8.t : 0u;
      }
      if constexpr (!EXACT) {
        u8.f += hi ? 0.0f : t.u8.f;
        other.u8.f += hi ? t.u8.f : 0.0f;
      }
    } else {
      part += hi ? A(0) : t.part;
      other.part += hi ? t.part : A(0);
    }
  }
  __device__ inline void flush() {
    if constexpr (U8) {
      u8.flush();
    } else {
      acc += static_cast<double>(part);
      part = A(0);
    }
  }
  // The wave's sum as 8 bytes (uint64, or the bits of a float64), valid in
  // every lane.
  __device__ inline uint64_t wave_bits() const {
    if constexpr (EXACT) return wave_sum(u8.exact);
    else return static_cast<uint64_t>(__double_as_longlong(wave_sum(U8 ? u8.wide : acc)));
  }
  // Adds two partials given as 8-byte patterns.
  __device__ static inline uint64_t add_bits(uint64_t x, uint64_t y) {
    if constexpr (EXACT) return x + y;
    else return static_cast<uint64_t>(__double_as_longlong(__longlong_as_double(x) + __longlong_as_double(y)));
  }
};

// --------------------------------------------------------------------------
// The single-launch finish of the exact uint8 sums (fa_gpu_pixel_reduce_once).
//
// Each workgroup adds its per-image sums, and its sum over the whole batch,
// to caller-owned accumulator words with ONE returning device-scope atomic
// per word that also counts the contribution: a word holds
// (sum << FIN_COUNT_BITS) + count.  The atomic's return value is the word
// before this add, so the workgroup whose add brings a word's count to
// gridDim.x holds that word's complete sum in registers (every other
// contribution is ordered before its own on that word) and finishes it
// itself: the mean, the dB, and a reset of the word to zero.  The image words
// and the batch word are added by different lanes of one instruction, so the
// call's tail is one atomic round trip.  No fence and no cache write-back is
// needed: nothing is read except through the returning atomics.  Each word
// sits on its own 128-byte line.
//
// The host allows the form only where every packed sum fits: the batch's
// n_total * max_term < 2^(64 - FIN_COUNT_BITS), which bounds the images too.
// --------------------------------------------------------------------------
constexpr int FIN_COUNT_BITS = 12;  // contributions per word: gridDim.x <= 4095
constexpr int FIN_STRIDE = 16;      // uint64 words between accumulators (128 bytes)
static_assert(FA_PIXEL_ACC_WORDS == (SWEEP_LDS_IMAGES + 1) * FIN_STRIDE,
              "the ABI's accumulator size");

struct SweepFin {
  uint64_t* acc;  // (n_images + 1) * FIN_STRIDE words, zero on entry and on exit
  double n_per_image, n_total, psnr_bias;
  double *out_per_image, *out_total, *out_psnr_per_image, *out_psnr_total;
};

// Thread-level: adds workgroup sum `t` to word `i` (image i, or the batch when
// i == n_images) and finishes the word when this is its last contribution.
__device__ inline void fin_word(const SweepFin& f, int i, int n_images, uint64_t t) {
  uint64_t* w = f.acc + static_cast<int64_t>(i) * FIN_STRIDE;
  const uint64_t old = __hip_atomic_fetch_add(w, (t << FIN_COUNT_BITS) + 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
  constexpr uint64_t CM = (uint64_t(1) << FIN_COUNT_BITS) - 1;
  if ((old & CM) + 1u != gridDim.x) return;
  __hip_atomic_store(w, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool batch = i == n_images;
  const double v = static_cast<double>((old >> FIN_COUNT_BITS) + t) /
                   (batch ? f.n_total : f.n_per_image);
  double* mean = batch ? f.out_total : (f.out_per_image ? f.out_per_image + i : nullptr);
  double* db = batch ? f.out_psnr_total
                     : (f.out_psnr_per_image ? f.out_psnr_per_image + i : nullptr);
  if (mean) *mean = v;
  if (f.psnr_bias != FA_PSNR_NONE && db) *db = f.psnr_bias - 10.0 * log10(v);
}

// FIN (exact uint8 sums, LDSP only): the workgroup finishes through
// fin_word instead of writing partials; each wave also keeps its sum over the
// whole batch for the batch word.
template <typename T, int OP, bool LDSP, int U = SWEEP_UNROLL, int NT = SWEEP_BLOCK,
          bool FIN = false>
__global__ __launch_bounds__(NT) void pix_sweep_kernel(
    const uint4* __restrict__ a, const uint4* __restrict__ b, int64_t nv, int n_images,
    double param, void* __restrict__ partial, SweepFin fin) {
  static_assert(!FIN || (LDSP && VecAcc<T, OP>::EXACT), "the one-launch finish takes exact sums");
  using Acc = VecAcc<T, OP>;
  constexpr int WPB = NT / WAVE;
  // LDSP: the waves' image sums wait in LDS and each workgroup writes one
  // partial per image at the end, partial[img * G + workgroup] (the finalize
  // then reads G instead of G * WPB per image); otherwise every wave writes
  // its own, partial[img * G * WPB + wave].
  __shared__ uint64_t s_p[LDSP ? SWEEP_LDS_IMAGES * WPB : 1];
  __shared__ uint64_t s_all[FIN ? WPB : 1];
  uint64_t wave_all = 0;  // FIN: this wave's sum over the batch
  const int64_t gs = static_cast<int64_t>(gridDim.x) * NT;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  const int64_t w0 = t0 - (threadIdx.x & (WAVE - 1));  // lane 0 of this wave
  const int64_t total = nv * n_images;
  const int64_t bpi = static_cast<int64_t>(gridDim.x) * WPB;
  const int wave = static_cast<int>(threadIdx.x) / WAVE;
  const int64_t wslot = static_cast<int64_t>(blockIdx.x) * WPB + wave;
  const bool lead = (threadIdx.x & (WAVE - 1)) == 0;
  const float p8 = static_cast<float>(param);
  const typename Acc::A p = static_cast<typename Acc::A>(param);

  Acc cur, nxt;        // this wave's image `img`, and the one after it
  int img = 0;         // wave-uniform
  int64_t edge = nv;   // first vector of image img + 1 (<= total while img < n_images)
  // A wave stops once it has written its last image: the batch's final round
  // can be short, and a wave past it would otherwise test its loads against
  // an edge beyond the end of the batch.  There is no barrier, so waves may
  // leave at different rounds.
  for (int64_t base = 0; img < n_images; base += U * gs) {  // wave-uniform
    uint4 xa[U], xb[U];
    if (base + (U - 1) * gs + w0 + (WAVE - 1) < edge) {
      // the wave's whole round lies in image img: no predication
#pragma unroll
      for (int u = 0; u < U; ++u) {
        xa[u] = ld_stream(a + base + u * gs + t0);
        xb[u] = ld_stream(b + base + u * gs + t0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) cur.add(xa[u], xb[u], p8, p);
      cur.flush();
    } else if (base + (U - 1) * gs + w0 + (WAVE - 1) < total) {
      // the round reaches the next image: lanes past the edge feed `nxt`
#pragma unroll
      for (int u = 0; u < U; ++u) {
        xa[u] = ld_stream(a + base + u * gs + t0);
        xb[u] = ld_stream(b + base + u * gs + t0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) cur.add_split(xa[u], xb[u], p8, p, base + u * gs + t0 >= edge, nxt);
      cur.flush();
      nxt.flush();
    } else {
      // the end of the batch: loads past it are skipped
      bool in[U], hi[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t v = base + u * gs + t0;
        in[u] = v < total;
        hi[u] = v >= edge;
        xa[u] = in[u] ? ld_stream(a + v) : make_uint4(0u, 0u, 0u, 0u);
        xb[u] = in[u] ? ld_stream(b + v) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // zero vectors add nothing, except Charbonnier's sqrt(0 + eps^2)
        if (OP != FA_OP_CHARB || in[u]) {
          if (hi[u]) nxt.add(xa[u], xb[u], p8, p);
          else cur.add(xa[u], xb[u], p8, p);
        }
      }
      cur.flush();
      nxt.flush();
    }
    // emit every image all of whose vectors this wave has passed
    const int64_t next = base + U * gs + w0;
    while (img < n_images && next >= edge) {
      const uint64_t bits = cur.wave_bits();
      if constexpr (FIN) wave_all += bits;
      if (lead) {
        if constexpr (LDSP) s_p[img * WPB + wave] = bits;
        else reinterpret_cast<uint64_t*>(partial)[img * bpi + wslot] = bits;
      }
      cur = nxt;
      nxt = Acc();
      ++img;
      edge += nv;
    }
  }
  if constexpr (FIN) {
    if (lead) s_all[wave] = wave_all;
  }
  if constexpr (LDSP) {
    __syncthreads();  // every wave has left the walk
    for (int i = static_cast<int>(threadIdx.x); i < n_images; i += NT) {
      uint64_t t = s_p[i * WPB];
#pragma unroll
      for (int w = 1; w < WPB; ++w) t = Acc::add_bits(t, s_p[i * WPB + w]);
      if constexpr (FIN) fin_word(fin, i, n_images, t);
      else reinterpret_cast<uint64_t*>(partial)[static_cast<int64_t>(i) * gridDim.x + blockIdx.x] = t;
    }
    if constexpr (FIN) {
      // the batch word, from a lane of the first wave that no image took
      // (n_images <= SWEEP_LDS_IMAGES < WAVE)
      const bool any_total = fin.out_total || (fin.psnr_bias != FA_PSNR_NONE && fin.out_psnr_total);
      if (static_cast<int>(threadIdx.x) == n_images && any_total) {
        uint64_t t = s_all[0];
#pragma unroll
        for (int w = 1; w < WPB; ++w) t += s_all[w];
        fin_word(fin, n_images, n_images, t);
      }
    }
  }
}

// One sweep launch of shape (U, NT) over G workgroups, or 0 when a round of
// it would span more than one image (the kernel touches at most two per
// round; smaller images take the per-image grid).  Returns the partial columns
// per image it writes: G for up to SWEEP_LDS_IMAGES images, G * NT / WAVE
// beyond (packed at that stride).
// With `fin` (exact sums of at most SWEEP_LDS_IMAGES images only) the launch
// finishes the call itself and returns -1.
template <typename T, int OP, int U, int NT>
static int launch_sweep_shape(hipStream_t st, const void* a, const void* b, int64_t n_images,
                              int64_t nv, int64_t G, double param, void* partial,
                              const SweepFin* fin) {
  if (nv < static_cast<int64_t>(U) * G * NT) return 0;
  const dim3 grid(static_cast<unsigned>(G));
  const uint4* va = static_cast<const uint4*>(a);
  const uint4* vb = static_cast<const uint4*>(b);
  const int ni = static_cast<int>(n_images);
  if constexpr (VecAcc<T, OP>::EXACT) {
    if (fin) {
      hipLaunchKernelGGL((pix_sweep_kernel<T, OP, true, U, NT, true>), grid, dim3(NT), 0, st,
                         va, vb, nv, ni, param, partial, *fin);
      return -1;
    }
  }
  if (n_images <= SWEEP_LDS_IMAGES) {
    hipLaunchKernelGGL((pix_sweep_kernel<T, OP, true, U, NT>), grid, dim3(NT), 0, st, va, vb,
                       nv, ni, param, partial, SweepFin{});
    return static_cast<int>(G);
  }
  hipLaunchKernelGGL((pix_sweep_kernel<T, OP, false, U, NT>), grid, dim3(NT), 0, st, va, vb, nv,
                     ni, param, partial, SweepFin{});
  return static_cast<int>(G * (NT / WAVE));
}

// Whether launch_sweep<T, OP> launches (the same tests, nothing launched).
template <typename T>
static bool sweep_applies(const void* a, const void* b, int64_t n_images, int64_t per,
                          int bpi) {
  constexpr int64_t E = 16 / static_cast<int64_t>(sizeof(T));
  const uintptr_t bases = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
  if ((bases & 15) != 0 || per % E != 0 || bpi % SWEEP_SLOTS_PER_CU != 0) return false;
  const int64_t nv = per / E;
  const int64_t G = bpi / SWEEP_SLOTS_PER_CU;
  if (std::is_same<T, uint8_t>::value && per * n_images < SWEEP_MANY_WAVES_BELOW)
    return nv >= G * SWEEP_MANY_BLOCK;
  return nv >= static_cast<int64_t>(SWEEP_UNROLL) * G * SWEEP_BLOCK;
}

// Launch of the sweep when it applies: 16-byte aligned bases, whole vectors
// per image, bpi a multiple of SWEEP_SLOTS_PER_CU (one workgroup per CU) and
// at least one round per image.  Returns the partial columns per image it
// writes, -1 when it finished the call through `fin`, or 0 when it does not
// apply and nothing was launched.
template <typename T, int OP>
static int launch_sweep(hipStream_t st, const void* a, const void* b, int64_t n_images,
                        int64_t per, int bpi, double param, void* partial,
                        const SweepFin* fin) {
  constexpr int64_t E = 16 / static_cast<int64_t>(sizeof(T));
  const uintptr_t bases = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
  if ((bases & 15) != 0 || per % E != 0 || bpi % SWEEP_SLOTS_PER_CU != 0) return 0;
  const int64_t nv = per / E;
  const int64_t G = bpi / SWEEP_SLOTS_PER_CU;
  if (std::is_same<T, uint8_t>::value && per * n_images < SWEEP_MANY_WAVES_BELOW)
    return launch_sweep_shape<T, OP, 1, SWEEP_MANY_BLOCK>(st, a, b, n_images, nv, G, param,
                                                          partial, fin);
  return launch_sweep_shape<T, OP, SWEEP_UNROLL, SWEEP_BLOCK>(st, a, b, n_images, nv, G, param,
                                                              partial, fin);
}

template <typename T>
static int launch_sweep_op(int op, hipStream_t st, const void* a, const void* b,
                           int64_t n_images, int64_t per, int bpi, double param,
                           void* partial, const SweepFin* fin = nullptr) {
  switch (op) {
    case FA_OP_MSE: return launch_sweep<T, FA_OP_MSE>(st, a, b, n_images, per, bpi, param, partial, fin);
    case FA_OP_L1: return launch_sweep<T, FA_OP_L1>(st, a, b, n_images, per, bpi, param, partial, fin);
    case FA_OP_CHARB: return launch_sweep<T, FA_OP_CHARB>(st, a, b, n_images, per, bpi, param, partial, nullptr);
    default: return launch_sweep<T, FA_OP_HUBER>(st, a, b, n_images, per, bpi, param, partial, nullptr);
  }
}

// --------------------------------------------------------------------------
// strided views and luma (fa_gpu_pixel_reduce_ex): a workgroup reduces an
// equal share of its image's (channel, row) space, lanes striding along a row
// (dwords for uint8 rows, realigned where a row starts off a 4-byte
// boundary).  With luma the difference of the two luma samples,
// kr dR + kg dG + kb dB (the offset cancels), is formed in float64 from the
// channel differences, and every term is float64.
// --------------------------------------------------------------------------
struct PixView {
  const void* a;
  const void* b;
  int64_t asn, asc, ash;  // element strides of image, channel, row
  int64_t bsn, bsc, bsh;
  int Cout, H, W;
  double kr, kg, kb;
  int bpi;
  double param;
  void* partial;
};

// Float views (float16 ... float64), one element per lane per row position.
template <typename T, int OP, bool LUMA>
__global__ __launch_bounds__(BLOCK) void pix_view_kernel(PixView v) {
  constexpr bool WIDE = LUMA || (OP != FA_OP_CHARB) || sizeof(T) == 8;
  using A = typename std::conditional<WIDE, double, float>::type;
  __shared__ double s_d[WAVES_PER_BLOCK];

  const int img = blockIdx.y;
  const int64_t R = static_cast<int64_t>(v.Cout) * v.H;
  const int64_t r0 = R * blockIdx.x / v.bpi;
  const int64_t r1 = R * (blockIdx.x + 1) / v.bpi;
  const T* ia = static_cast<const T*>(v.a) + img * v.asn;
  const T* ib = static_cast<const T*>(v.b) + img * v.bsn;
  const A p = static_cast<A>(v.param);

  double acc = 0.0;
  for (int64_t rr = r0; rr < r1; ++rr) {  // uniform
    const int c = static_cast<int>(rr / v.H);
    const int row = static_cast<int>(rr - static_cast<int64_t>(c) * v.H);
    if constexpr (LUMA) {
      const T* pa = ia + row * v.ash;
      const T* pb = ib + row * v.bsh;
      double part = 0.0;
      for (int j = threadIdx.x; j < v.W; j += BLOCK) {
        const double dr = Elem<T>::d(pa[j]) - Elem<T>::d(pb[j]);
        const double dg = Elem<T>::d(pa[v.asc + j]) - Elem<T>::d(pb[v.bsc + j]);
        const double db = Elem<T>::d(pa[2 * v.asc + j]) - Elem<T>::d(pb[2 * v.bsc + j]);
        part += pix_term<OP, double>(fma(v.kb, db, fma(v.kg, dg, v.kr * dr)), p);
      }
      acc += part;
    } else {
      const T* pa = ia + c * v.asc + row * v.ash;
      const T* pb = ib + c * v.bsc + row * v.bsh;
      A part = A(0);
      for (int j = threadIdx.x; j < v.W; j += BLOCK)
        part += pix_term<OP, A>(load_as<A>(pa, j) - load_as<A>(pb, j), p);
      acc += static_cast<double>(part);
    }
  }
  const double t = block_sum(acc, s_d);
  if (threadIdx.x == 0) reinterpret_cast<double*>(v.partial)[static_cast<int64_t>(img) * v.bpi + blockIdx.x] = t;
}

// uint8 views: crops at any byte offset, with or without luma.  A row is read
// as dwords -- realigned with v_alignbyte when it does not start on a 4-byte
// boundary, since the aligned dword holding any byte of the row is mapped --
// and a lane issues the loads of VR rows x VQ dwords (rows up to 4 KiB in one
// step) before it sums any, so enough bytes are in flight: one dword load per
// row at a time left this kernel latency bound (a 4-byte aligned crop of
// configs[2] took 85 us, a byte-offset one 204 us).  With luma the three
// channels' dwords are read and kr dR + kg dG + kb dB is formed per pixel in
// float64 (the luma offset cancels).
constexpr int PIX_VQ = 4;  // dwords per lane per row and step
constexpr int PIX_VIEW_WG_PER_CU = 4;

// A row at address `row` = m (mod 4) is read as the aligned dwords
// al[j] = (row - m)[4j, 4j + 4): the bytes [4j, 4j + 4) of the row are
// alignbyte(al[j + 1], al[j], m).  Lanes of a wave hold consecutive j, so
// al[j + 1] is the next lane's dword (a DPP move), and only lane 63 loads it
// itself.  The aligned dwords up to index nq = W / 4 each hold a byte of the
// row, so they are mapped.  All loads of a step are issued before the first
// DPP move: a move per load, between the loads, made the compiler wait for
// each load in turn (crop at a byte offset: 355 us against 232).
template <int OP, bool LUMA>
__global__ __launch_bounds__(BLOCK) void pix_view_u8_kernel(PixView v) {
  constexpr bool EXACT = !LUMA && (OP == FA_OP_MSE || OP == FA_OP_L1);
  constexpr int CH = LUMA ? 3 : 1;
  constexpr int VR = LUMA ? 1 : 2;  // rows per step
  __shared__ uint64_t s_u[WAVES_PER_BLOCK];
  __shared__ double s_d[WAVES_PER_BLOCK];

  const int img = blockIdx.y;
  const int64_t R = static_cast<int64_t>(v.Cout) * v.H;
  const int64_t r0 = R * blockIdx.x / v.bpi;
  const int64_t r1 = R * (blockIdx.x + 1) / v.bpi;
  const uint8_t* ia = static_cast<const uint8_t*>(v.a) + img * v.asn;
  const uint8_t* ib = static_cast<const uint8_t*>(v.b) + img * v.bsn;
  const float p8 = static_cast<float>(v.param);
  const double pd = v.param;
  const int nq = v.W / 4;          // whole dwords per row
  const int tail = v.W - 4 * nq;   // trailing bytes per row

  U8Lane<OP> lane8;   // without luma
  double acc = 0.0;   // with luma
  // the luma term of byte k of the dwords xa / xb of the three channels
  auto luma_px = [&](const uint32_t (&xa)[3], const uint32_t (&xb)[3], int k) {
    double d[3];
#pragma unroll
    for (int ch = 0; ch < 3; ++ch)
      d[ch] = static_cast<double>(static_cast<int>((xa[ch] >> (8 * k)) & 0xffu) -
                                  static_cast<int>((xb[ch] >> (8 * k)) & 0xffu));
    return pix_term<OP, double>(fma(v.kb, d[2], fma(v.kg, d[1], v.kr * d[0])), pd);
  };

  for (int64_t rr = r0; rr < r1; rr += VR) {  // uniform
    const uint8_t* pa[VR][CH];
    const uint8_t* pb[VR][CH];
    uint32_t ma[VR][CH], mb[VR][CH];
    bool rv[VR];
#pragma unroll
    for (int q = 0; q < VR; ++q) {
      rv[q] = rr + q < r1;
      const int64_t rq = rv[q] ? rr + q : rr;
      const int c = static_cast<int>(rq / v.H);
      const int row = static_cast<int>(rq - static_cast<int64_t>(c) * v.H);
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        const int cc = LUMA ? ch : c;
        pa[q][ch] = ia + cc * v.asc + row * v.ash;
        pb[q][ch] = ib + cc * v.bsc + row * v.bsh;
        ma[q][ch] = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(pa[q][ch]) & 3);
        mb[q][ch] = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(pb[q][ch]) & 3);
      }
    }
    for (int j0 = 0; j0 < nq; j0 += PIX_VQ * BLOCK) {  // uniform; one step for rows <= 4 KiB
      uint32_t xa[VR][PIX_VQ][CH], xb[VR][PIX_VQ][CH];
      uint32_t ha[VR][PIX_VQ][CH], hb[VR][PIX_VQ][CH];  // lane 63's al[j + 1]
      bool ok[VR][PIX_VQ];
      const bool last_lane = (threadIdx.x & (WAVE - 1)) == WAVE - 1;
      // every load of the step first ...
#pragma unroll
      for (int q = 0; q < VR; ++q) {
#pragma unroll
        for (int u = 0; u < PIX_VQ; ++u) {
          const int j = j0 + u * BLOCK + static_cast<int>(threadIdx.x);
          ok[q][u] = rv[q] && j < nq;
          const bool feed = rv[q] && j == nq;  // loads only for its neighbour
#pragma unroll
          for (int ch = 0; ch < CH; ++ch) {
            const uint32_t* wa = reinterpret_cast<const uint32_t*>(pa[q][ch] - ma[q][ch]);
            const uint32_t* wb = reinterpret_cast<const uint32_t*>(pb[q][ch] - mb[q][ch]);
            xa[q][u][ch] = (ok[q][u] || (feed && ma[q][ch])) ? wa[j] : 0u;
            xb[q][u][ch] = (ok[q][u] || (feed && mb[q][ch])) ? wb[j] : 0u;
            ha[q][u][ch] = (last_lane && ok[q][u] && ma[q][ch]) ? wa[j + 1] : 0u;
            hb[q][u][ch] = (last_lane && ok[q][u] && mb[q][ch]) ? wb[j + 1] : 0u;
          }
        }
      }
      // ... then the realignment of rows off a 4-byte boundary (m uniform)
#pragma unroll
      for (int q = 0; q < VR; ++q) {
#pragma unroll
        for (int u = 0; u < PIX_VQ; ++u) {
#pragma unroll
          for (int ch = 0; ch < CH; ++ch) {
            if (ma[q][ch]) {
              const uint32_t nx = static_cast<uint32_t>(wave_next(static_cast<int>(xa[q][u][ch])));
              const uint32_t hi = last_lane ? ha[q][u][ch] : nx;
              xa[q][u][ch] = ok[q][u] ? __builtin_amdgcn_alignbyte(hi, xa[q][u][ch], ma[q][ch]) : 0u;
            }
            if (mb[q][ch]) {
              const uint32_t nx = static_cast<uint32_t>(wave_next(static_cast<int>(xb[q][u][ch])));
              const uint32_t hi = last_lane ? hb[q][u][ch] : nx;
              xb[q][u][ch] = ok[q][u] ? __builtin_amdgcn_alignbyte(hi, xb[q][u][ch], mb[q][ch]) : 0u;
            }
          }
        }
      }
      if constexpr (LUMA) {
        double part = 0.0;
#pragma unroll
        for (int u = 0; u < PIX_VQ; ++u) {
          if (ok[0][u]) {
            const uint32_t a3[3] = {xa[0][u][0], xa[0][u][1], xa[0][u][2]};
            const uint32_t b3[3] = {xb[0][u][0], xb[0][u][1], xb[0][u][2]};
#pragma unroll
            for (int k = 0; k < 4; ++k) part += luma_px(a3, b3, k);
          }
        }
        acc += part;
      } else {
#pragma unroll
        for (int q = 0; q < VR; ++q) {
#pragma unroll
          for (int u = 0; u < PIX_VQ; ++u) {
            // zeros add nothing, except Charbonnier's sqrt(0 + eps^2)
            if (EXACT || ok[q][u]) lane8.dword(xa[q][u][0], xb[q][u][0], p8);
          }
        }
        lane8.flush();  // at most VR * PIX_VQ = 8 dwords since the last flush
      }
    }
    if (static_cast<int>(threadIdx.x) < tail) {  // the row's last W % 4 bytes
      const int j = 4 * nq + static_cast<int>(threadIdx.x);
#pragma unroll
      for (int q = 0; q < VR; ++q) {
        if (rv[q]) {
          if constexpr (LUMA) {
            const uint32_t a3[3] = {pa[q][0][j], pa[q][1][j], pa[q][2][j]};
            const uint32_t b3[3] = {pb[q][0][j], pb[q][1][j], pb[q][2][j]};
            acc += luma_px(a3, b3, 0);
          } else {
            lane8.byte(pa[q][0][j], pb[q][0][j], p8);
          }
        }
      }
    }
  }

  const int64_t slot = static_cast<int64_t>(img) * v.bpi + blockIdx.x;
  if constexpr (EXACT) {
    const uint64_t t = block_sum(lane8.exact, s_u);
    if (threadIdx.x == 0) reinterpret_cast<uint64_t*>(v.partial)[slot] = t;
  } else {
    if constexpr (!LUMA) {
      lane8.flush();
      acc += lane8.wide;
    }
    const double t = block_sum(acc, s_d);
    if (threadIdx.x == 0) reinterpret_cast<double*>(v.partial)[slot] = t;
  }
}

template <typename T, int OP, bool LUMA>
static void launch_view(dim3 grid, hipStream_t st, const PixView& v) {
  if constexpr (std::is_same<T, uint8_t>::value)
    hipLaunchKernelGGL((pix_view_u8_kernel<OP, LUMA>), grid, dim3(BLOCK), 0, st, v);
  else
    hipLaunchKernelGGL((pix_view_kernel<T, OP, LUMA>), grid, dim3(BLOCK), 0, st, v);
}

template <typename T, bool LUMA>
static void launch_view_op(int op, dim3 grid, hipStream_t st, const PixView& v) {
  switch (op) {
    case FA_OP_MSE: launch_view<T, FA_OP_MSE, LUMA>(grid, st, v); break;
    case FA_OP_L1: launch_view<T, FA_OP_L1, LUMA>(grid, st, v); break;
    case FA_OP_CHARB: launch_view<T, FA_OP_CHARB, LUMA>(grid, st, v); break;
    default: launch_view<T, FA_OP_HUBER, LUMA>(grid, st, v); break;
  }
}

template <bool LUMA>
static int launch_view_dtype(int dtype, int op, dim3 grid, hipStream_t st, const PixView& v) {
  switch (dtype) {
    case FA_U8: launch_view_op<uint8_t, LUMA>(op, grid, st, v); break;
    case FA_F16: launch_view_op<half_t, LUMA>(op, grid, st, v); break;
    case FA_BF16: launch_view_op<bf16_t, LUMA>(op, grid, st, v); break;
    case FA_F32: launch_view_op<float, LUMA>(op, grid, st, v); break;
    case FA_F64: launch_view_op<double, LUMA>(op, grid, st, v); break;
    default: return FA_E_DTYPE;
  }
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// --------------------------------------------------------------------------
// finalize: block r < nrows reduces row r, block nrows reduces everything.
// Means are divisions by the count (reference fa_cuda.cu:177-181); a PSNR is
// psnr_bias - 10*log10(mean), +inf for a zero mean (reference :203-208).
// --------------------------------------------------------------------------
// The finalize's workgroup size: the partials come from other XCDs' L2s, so
// every round of dependent loads waits the full memory latency; with 1024
// lanes and 8 loads in flight per lane the total of a configs[2] PSNR
// (8 x 2048 partials) is two rounds (256 lanes took 5.5 us for it).
constexpr int FIN_BLOCK = 1024;

// Sum of p[begin, end) over the workgroup's lanes (this lane's share), the
// loads of 8 strides issued together.
template <typename V>
__device__ inline V strided_sum(const V* __restrict__ p, int64_t begin, int64_t end) {
  constexpr int FU = 8;
  V acc[FU];
#pragma unroll
  for (int u = 0; u < FU; ++u) acc[u] = V(0);
  int64_t i = begin + threadIdx.x;
  for (; i + (FU - 1) * FIN_BLOCK < end; i += FU * FIN_BLOCK) {
    V x[FU];
#pragma unroll
    for (int u = 0; u < FU; ++u) x[u] = p[i + u * FIN_BLOCK];
#pragma unroll
    for (int u = 0; u < FU; ++u) acc[u] += x[u];
  }
#pragma unroll
  for (int u = 0; u < FU; ++u)
    if (i + u * FIN_BLOCK < end) acc[u] += p[i + u * FIN_BLOCK];
  V t = acc[0];
#pragma unroll
  for (int u = 1; u < FU; ++u) t += acc[u];
  return t;
}

__global__ __launch_bounds__(FIN_BLOCK) void finalize_kernel(
    const void* __restrict__ partial, int exact, int nrows, int ncols,
    double n_per_row, double n_total, double psnr_bias,
    double* __restrict__ out_per_row, double* __restrict__ out_total,
    double* __restrict__ out_psnr_per_row, double* __restrict__ out_psnr_total) {
  __shared__ uint64_t s_u[FIN_BLOCK / WAVE];
  __shared__ double s_d[FIN_BLOCK / WAVE];
  const int row = blockIdx.x;
  const bool is_total = (row == nrows);
  const int64_t begin = is_total ? 0 : static_cast<int64_t>(row) * ncols;
  const int64_t end = is_total ? static_cast<int64_t>(nrows) * ncols : begin + ncols;

  double s;
  if (exact) {
    const uint64_t t = strided_sum(reinterpret_cast<const uint64_t*>(partial), begin, end);
    s = static_cast<double>(block_sum<uint64_t, FIN_BLOCK>(t, s_u));
  } else {
    s = block_sum<double, FIN_BLOCK>(
        strided_sum(reinterpret_cast<const double*>(partial), begin, end), s_d);
  }
  if (threadIdx.x == 0) {
    const double v = s / (is_total ? n_total : n_per_row);
    if (is_total) {
      if (out_total) *out_total = v;
    } else if (out_per_row) {
      out_per_row[row] = v;
    }
    if (psnr_bias != FA_PSNR_NONE) {
      const double db = psnr_bias - 10.0 * log10(v);
      if (is_total) {
        if (out_psnr_total) *out_psnr_total = db;
      } else if (out_psnr_per_row) {
        out_psnr_per_row[row] = db;
      }
    }
  }
}

int launch_finalize(const void* partial, bool exact, int nrows, int ncols,
                    double n_per_row, double n_total, double psnr_bias,
                    double* out_per_row, double* out_total,
                    double* out_psnr_per_row, double* out_psnr_total,
                    hipStream_t st) {
  if (!out_per_row && !out_total && !out_psnr_per_row && !out_psnr_total)
    return FA_OK;
  hipLaunchKernelGGL(finalize_kernel, dim3(nrows + 1), dim3(FIN_BLOCK), 0, st,
                     partial, exact ? 1 : 0, nrows, ncols, n_per_row, n_total,
                     psnr_bias, out_per_row, out_total, out_psnr_per_row,
                     out_psnr_total);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

template <int OP>
static void launch_u8(int vec, dim3 grid, hipStream_t st, const void* a,
                      const void* b, int64_t per, int bpi, float p,
                      void* partial) {
  const uint8_t* ua = static_cast<const uint8_t*>(a);
  const uint8_t* ub = static_cast<const uint8_t*>(b);
  if (vec == 16)
    hipLaunchKernelGGL((pix_u8_kernel<OP, 16>), grid, dim3(BLOCK), 0, st, ua, ub, per, bpi, p, partial);
  else if (vec == 4)
    hipLaunchKernelGGL((pix_u8_kernel<OP, 4>), grid, dim3(BLOCK), 0, st, ua, ub, per, bpi, p, partial);
  else
    hipLaunchKernelGGL((pix_u8_kernel<OP, 1>), grid, dim3(BLOCK), 0, st, ua, ub, per, bpi, p, partial);
}

template <typename T, int OP>
static void launch_float(bool vec, dim3 grid, hipStream_t st, const void* a,
                         const void* b, int64_t per, int bpi, double p,
                         double* partial) {
  const T* ta = static_cast<const T*>(a);
  const T* tb = static_cast<const T*>(b);
  if (vec)
    hipLaunchKernelGGL((pix_float_kernel<T, OP, true>), grid, dim3(BLOCK), 0, st, ta, tb, per, bpi, p, partial);
  else
    hipLaunchKernelGGL((pix_float_kernel<T, OP, false>), grid, dim3(BLOCK), 0, st, ta, tb, per, bpi, p, partial);
}

template <typename T>
static void launch_float_op(int op, bool vec, dim3 grid, hipStream_t st,
                            const void* a, const void* b, int64_t per, int bpi,
                            double p, double* partial) {
  switch (op) {
    case FA_OP_MSE: launch_float<T, FA_OP_MSE>(vec, grid, st, a, b, per, bpi, p, partial); break;
    case FA_OP_L1: launch_float<T, FA_OP_L1>(vec, grid, st, a, b, per, bpi, p, partial); break;
    case FA_OP_CHARB: launch_float<T, FA_OP_CHARB>(vec, grid, st, a, b, per, bpi, p, partial); break;
    default: launch_float<T, FA_OP_HUBER>(vec, grid, st, a, b, per, bpi, p, partial); break;
  }
}

}  // namespace fa

using namespace fa;

extern "C" {

// reference: fa_cuda.cu:1065-1076 (fa_cuda_pixel_workspace)
FA_API int fa_gpu_pixel_workspace(int64_t n_images, int64_t n_per_image,
                                  int device, int* out_bpi) {
  if (!out_bpi) return FA_E_ARG;
  if (n_images <= 0 || n_per_image <= 0 || n_images > 65535) return FA_E_SHAPE;
  const int64_t cus = cu_count(device);
  if (n_per_image >= PIX_SWEEP_MIN_ELEMS) {
    // the sweep: one workgroup per CU, one partial per wave of its larger shape
    *out_bpi = static_cast<int>(cus * SWEEP_SLOTS_PER_CU);
    return FA_OK;
  }
  const int64_t by_device = std::max<int64_t>(1, cus * PIX_WG_PER_CU / n_images);
  const int64_t per_wg = static_cast<int64_t>(BLOCK) * PIX_MIN_ELEMS_PER_THREAD;
  const int64_t by_size = std::max<int64_t>(1, (n_per_image + per_wg - 1) / per_wg);
  *out_bpi = static_cast<int>(std::min(by_device, by_size));
  return FA_OK;
}

// reference: fa_cuda.cu:1078-1156 (fa_cuda_pixel_reduce)
FA_API int fa_gpu_pixel_reduce(const void* a, const void* b, int dtype,
                               int64_t n_images, int64_t n_per_image, int op,
                               double param, double psnr_bias, double* partial,
                               int bpi, double* out_per_image,
                               double* out_total, double* out_psnr_per_image,
                               double* out_psnr_total, int device,
                               void* stream) {
  return fa_gpu_pixel_reduce_once(a, b, dtype, n_images, n_per_image, op, param, psnr_bias,
                                  partial, bpi, nullptr, out_per_image, out_total,
                                  out_psnr_per_image, out_psnr_total, device, stream);
}

// No counterpart in the reference: fa_gpu_pixel_reduce whose exact uint8 sums
// (MSE / PSNR / L1 over the sweep) finish inside the sweep launch through
// `acc`, a caller-owned zeroed buffer the call leaves zeroed.
FA_API int fa_gpu_pixel_reduce_once(const void* a, const void* b, int dtype,
                                    int64_t n_images, int64_t n_per_image, int op,
                                    double param, double psnr_bias, double* partial,
                                    int bpi, uint64_t* acc, double* out_per_image,
                                    double* out_total, double* out_psnr_per_image,
                                    double* out_psnr_total, int device, void* stream) {
  if (!a || !b || (!partial && !acc)) return FA_E_ARG;
  if (op < 0 || op > 3) return FA_E_OP;
  if (n_images <= 0 || n_per_image <= 0 || bpi <= 0) return FA_E_SHAPE;
  if (n_images > 65535 || static_cast<int64_t>(bpi) * BLOCK > INT32_MAX) return FA_E_SHAPE;
  const dim3 grid(static_cast<unsigned>(bpi), static_cast<unsigned>(n_images));
  const uintptr_t rel = reinterpret_cast<uintptr_t>(a) - reinterpret_cast<uintptr_t>(b);

  // the one-launch finish: exact uint8 sums, a wanted output, and every
  // packed word within its bits (the batch's sum below 2^52, so each image's
  // is too; the contribution count below 2^12)
  SweepFin fin = {};
  const SweepFin* pfin = nullptr;
  const bool want = out_per_image || out_total ||
                    (psnr_bias != FA_PSNR_NONE && (out_psnr_per_image || out_psnr_total));
  if (acc && want && dtype == FA_U8 && (op == FA_OP_MSE || op == FA_OP_L1) &&
      n_images <= SWEEP_LDS_IMAGES && bpi / SWEEP_SLOTS_PER_CU < (1 << FIN_COUNT_BITS)) {
    const int64_t term = op == FA_OP_MSE ? 255 * 255 : 255;
    const int64_t lim = (int64_t(1) << (64 - FIN_COUNT_BITS)) / term;
    if (n_per_image < lim / n_images) {
      fin.acc = acc;
      fin.n_per_image = static_cast<double>(n_per_image);
      fin.n_total = static_cast<double>(n_per_image) * static_cast<double>(n_images);
      fin.psnr_bias = psnr_bias;
      fin.out_per_image = out_per_image;
      fin.out_total = out_total;
      fin.out_psnr_per_image = out_psnr_per_image;
      fin.out_psnr_total = out_psnr_total;
      pfin = &fin;
    }
  }
  // a null workspace is enough only for the one-launch form
  if (!partial && !(pfin && sweep_applies<uint8_t>(a, b, n_images, n_per_image, bpi)))
    return FA_E_ARG;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);

  bool exact = false;
  int swept = 0;  // partial columns per image the sweep wrote, 0 if it did not run
  switch (dtype) {
    case FA_U8:
      swept = launch_sweep_op<uint8_t>(op, st, a, b, n_images, n_per_image, bpi, param, partial,
                                       pfin);
      if (swept < 0) {  // finished inside the sweep
        FA_LAUNCH_CHECK();
        return FA_OK;
      }
      break;
    case FA_F16: swept = launch_sweep_op<half_t>(op, st, a, b, n_images, n_per_image, bpi, param, partial); break;
    case FA_BF16: swept = launch_sweep_op<bf16_t>(op, st, a, b, n_images, n_per_image, bpi, param, partial); break;
    case FA_F32: swept = launch_sweep_op<float>(op, st, a, b, n_images, n_per_image, bpi, param, partial); break;
    case FA_F64: swept = launch_sweep_op<double>(op, st, a, b, n_images, n_per_image, bpi, param, partial); break;
    default: return FA_E_DTYPE;
  }
  if (swept) {
    exact = dtype == FA_U8 && (op == FA_OP_MSE || op == FA_OP_L1);
  } else if (dtype == FA_U8) {
    const int vec = (rel & 15) == 0 ? 16 : ((rel & 3) == 0 ? 4 : 1);
    const float p = static_cast<float>(param);
    exact = (op == FA_OP_MSE || op == FA_OP_L1);
    switch (op) {
      case FA_OP_MSE: launch_u8<FA_OP_MSE>(vec, grid, st, a, b, n_per_image, bpi, p, partial); break;
      case FA_OP_L1: launch_u8<FA_OP_L1>(vec, grid, st, a, b, n_per_image, bpi, p, partial); break;
      case FA_OP_CHARB: launch_u8<FA_OP_CHARB>(vec, grid, st, a, b, n_per_image, bpi, p, partial); break;
      default: launch_u8<FA_OP_HUBER>(vec, grid, st, a, b, n_per_image, bpi, p, partial); break;
    }
  } else {
    const bool vec = (rel & 15) == 0;
    switch (dtype) {
      case FA_F16: launch_float_op<half_t>(op, vec, grid, st, a, b, n_per_image, bpi, param, partial); break;
      case FA_BF16: launch_float_op<bf16_t>(op, vec, grid, st, a, b, n_per_image, bpi, param, partial); break;
      case FA_F32: launch_float_op<float>(op, vec, grid, st, a, b, n_per_image, bpi, param, partial); break;
      case FA_F64: launch_float_op<double>(op, vec, grid, st, a, b, n_per_image, bpi, param, partial); break;
      default: return FA_E_DTYPE;
    }
  }
  FA_LAUNCH_CHECK();

  const double n_each = static_cast<double>(n_per_image);
  return launch_finalize(partial, exact, static_cast<int>(n_images), swept ? swept : bpi,
                         n_each, n_each * static_cast<double>(n_images), psnr_bias,
                         out_per_image, out_total, out_psnr_per_image, out_psnr_total, st);
}

// No counterpart in the reference, which materialises a float32 luma plane
// (functional.py:267-271) and copies crops contiguous (backend.py:346,482).
FA_API int fa_gpu_pixel_reduce_ex(const void* a, const void* b, int dtype, int64_t n_images,
                                  int C, int H, int W, const int64_t* a_strides,
                                  const int64_t* b_strides, const double* luma, int op,
                                  double param, double psnr_bias, double* partial, int bpi,
                                  double* out_per_image, double* out_total,
                                  double* out_psnr_per_image, double* out_psnr_total,
                                  int device, void* stream) {
  if (!a || !b || !partial) return FA_E_ARG;
  if (op < 0 || op > 3) return FA_E_OP;
  if (dtype < FA_U8 || dtype > FA_F64) return FA_E_DTYPE;
  if (n_images <= 0 || n_images > 65535 || C <= 0 || H <= 0 || W <= 0 || bpi <= 0)
    return FA_E_SHAPE;
  if (luma && C != 3) return FA_E_SHAPE;
  const int64_t plane = static_cast<int64_t>(H) * W;
  const int64_t va[3] = {a_strides ? a_strides[0] : plane * C, a_strides ? a_strides[1] : plane,
                         a_strides ? a_strides[2] : W};
  const int64_t vb[3] = {b_strides ? b_strides[0] : plane * C, b_strides ? b_strides[1] : plane,
                         b_strides ? b_strides[2] : W};
  for (int i = 0; i < 3; ++i)
    if (va[i] < 0 || vb[i] < 0) return FA_E_SHAPE;
  if (va[2] < W || vb[2] < W) return FA_E_SHAPE;  // rows may not overlap

  PixView v = {};
  v.a = a;
  v.b = b;
  v.asn = va[0];
  v.asc = va[1];
  v.ash = va[2];
  v.bsn = vb[0];
  v.bsc = vb[1];
  v.bsh = vb[2];
  v.Cout = luma ? 1 : C;
  v.H = H;
  v.W = W;
  if (luma) {
    v.kr = luma[0];
    v.kg = luma[1];
    v.kb = luma[2];
  }
  // The view kernels take about 4 workgroups per CU, whatever the workspace
  // allows: each uses the first `cols` partial slots of its image, packed.
  // Measured at 8x3x2160x3840 uint8 (1 / 2 / 4 / 8 workgroups per CU): crop
  // border 4, 156 / 95 / 77 / 83 us; luma, 148 / 92 / 77 / 79 us; and 91 us
  // and 126 us with all 2048 columns of the sweep's workspace.
  const int64_t cus = cu_count(device);
  const int cols = static_cast<int>(std::max<int64_t>(
      1, std::min<int64_t>(bpi, std::max<int64_t>(1, cus * PIX_VIEW_WG_PER_CU / n_images))));
  v.bpi = cols;
  v.param = param;
  v.partial = partial;

  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(cols), static_cast<unsigned>(n_images));
  const int rc = luma ? launch_view_dtype<true>(dtype, op, grid, st, v)
                      : launch_view_dtype<false>(dtype, op, grid, st, v);
  if (rc != FA_OK) return rc;
  const bool exact = dtype == FA_U8 && !luma && (op == FA_OP_MSE || op == FA_OP_L1);
  const double n_each = static_cast<double>(v.Cout) * plane;
  return launch_finalize(partial, exact, static_cast<int>(n_images), cols, n_each,
                         n_each * static_cast<double>(n_images), psnr_bias, out_per_image,
                         out_total, out_psnr_per_image, out_psnr_total, st);
}

}  // extern "C"
