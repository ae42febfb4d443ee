// Pixel losses on gfx950: MSE / L1 / Charbonnier / Huber, and PSNR folded
// into the final reduction.
//
// Behaviour follows the reference's pixel_kernel_u8 / pixel_kernel /
// finalize_kernel (reference: fa_cuda.cu:182-210, 252-359, 1065-1156):
// per-image sums, divided (never multiplied by a reciprocal) by the element
// count, optionally turned into dB as psnr_bias - 10*log10(mse).
//
// The design is CDNA4's own:
//   * uint8 is streamed with 16-byte global loads (global_load_dwordx4), four
//     vectors in flight per lane per tensor, so a 256-CU part keeps enough
//     bytes outstanding to sit on the HBM roofline.
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
// strided views and luma (fa_gpu_pixel_reduce_ex): a workgroup reduces an
// equal share of its image's (channel, row) space, lanes striding along a row
// (dwords for 4-byte aligned uint8 rows).  With luma the difference of the
// two luma samples, kr dR + kg dG + kb dB (the offset cancels), is formed in
// float64 from the channel differences, and every term is float64.
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

template <typename T, int OP, bool LUMA, int V>
__global__ __launch_bounds__(BLOCK) void pix_view_kernel(PixView v) {
  constexpr bool U8 = std::is_same<T, uint8_t>::value;
  constexpr bool EXACT = U8 && !LUMA && (OP == FA_OP_MSE || OP == FA_OP_L1);
  constexpr bool WIDE = LUMA || (OP != FA_OP_CHARB) || sizeof(T) == 8;
  using A = typename std::conditional<WIDE, double, float>::type;
  __shared__ uint64_t s_u[WAVES_PER_BLOCK];
  __shared__ double s_d[WAVES_PER_BLOCK];

  const int img = blockIdx.y;
  const int64_t R = static_cast<int64_t>(v.Cout) * v.H;
  const int64_t r0 = R * blockIdx.x / v.bpi;
  const int64_t r1 = R * (blockIdx.x + 1) / v.bpi;
  const T* ia = static_cast<const T*>(v.a) + img * v.asn;
  const T* ib = static_cast<const T*>(v.b) + img * v.bsn;
  const A p = static_cast<A>(v.param);

  U8Lane<OP> lane8;   // uint8 without luma
  double acc = 0.0;   // everything else
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
      if constexpr (U8 && V == 4) {
        const uint32_t* wa = reinterpret_cast<const uint32_t*>(pa);
        const uint32_t* wb = reinterpret_cast<const uint32_t*>(pb);
        for (int j = threadIdx.x; j < v.W / 4; j += BLOCK) {
          lane8.dword(wa[j], wb[j], static_cast<float>(v.param));
          lane8.flush();
        }
      } else if constexpr (U8) {
        for (int j = threadIdx.x; j < v.W; j += BLOCK) lane8.byte(pa[j], pb[j], static_cast<float>(v.param));
      } else {
        A part = A(0);
        for (int j = threadIdx.x; j < v.W; j += BLOCK)
          part += pix_term<OP, A>(load_as<A>(pa, j) - load_as<A>(pb, j), p);
        acc += static_cast<double>(part);
      }
    }
  }

  const int64_t slot = static_cast<int64_t>(img) * v.bpi + blockIdx.x;
  if constexpr (EXACT) {
    const uint64_t t = block_sum(lane8.exact, s_u);
    if (threadIdx.x == 0) reinterpret_cast<uint64_t*>(v.partial)[slot] = t;
  } else {
    if constexpr (U8 && !LUMA) {
      lane8.flush();
      acc += lane8.wide;
    }
    const double t = block_sum(acc, s_d);
    if (threadIdx.x == 0) reinterpret_cast<double*>(v.partial)[slot] = t;
  }
}

template <typename T, int OP, bool LUMA>
static void launch_view(bool dw, dim3 grid, hipStream_t st, const PixView& v) {
  if (dw)
    hipLaunchKernelGGL((pix_view_kernel<T, OP, LUMA, 4>), grid, dim3(BLOCK), 0, st, v);
  else
    hipLaunchKernelGGL((pix_view_kernel<T, OP, LUMA, 1>), grid, dim3(BLOCK), 0, st, v);
}

template <typename T, bool LUMA>
static void launch_view_op(int op, bool dw, dim3 grid, hipStream_t st, const PixView& v) {
  switch (op) {
    case FA_OP_MSE: launch_view<T, FA_OP_MSE, LUMA>(dw, grid, st, v); break;
    case FA_OP_L1: launch_view<T, FA_OP_L1, LUMA>(dw, grid, st, v); break;
    case FA_OP_CHARB: launch_view<T, FA_OP_CHARB, LUMA>(dw, grid, st, v); break;
    default: launch_view<T, FA_OP_HUBER, LUMA>(dw, grid, st, v); break;
  }
}

template <bool LUMA>
static int launch_view_dtype(int dtype, int op, bool dw, dim3 grid, hipStream_t st,
                             const PixView& v) {
  switch (dtype) {
    case FA_U8: launch_view_op<uint8_t, LUMA>(op, dw, grid, st, v); break;
    case FA_F16: launch_view_op<half_t, LUMA>(op, false, grid, st, v); break;
    case FA_BF16: launch_view_op<bf16_t, LUMA>(op, false, grid, st, v); break;
    case FA_F32: launch_view_op<float, LUMA>(op, false, grid, st, v); break;
    case FA_F64: launch_view_op<double, LUMA>(op, false, grid, st, v); break;
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
__global__ __launch_bounds__(BLOCK) void finalize_kernel(
    const void* __restrict__ partial, int exact, int nrows, int ncols,
    double n_per_row, double n_total, double psnr_bias,
    double* __restrict__ out_per_row, double* __restrict__ out_total,
    double* __restrict__ out_psnr_per_row, double* __restrict__ out_psnr_total) {
  __shared__ uint64_t s_u[WAVES_PER_BLOCK];
  __shared__ double s_d[WAVES_PER_BLOCK];
  const int row = blockIdx.x;
  const bool is_total = (row == nrows);
  const int64_t begin = is_total ? 0 : static_cast<int64_t>(row) * ncols;
  const int64_t end = is_total ? static_cast<int64_t>(nrows) * ncols : begin + ncols;

  double s;
  if (exact) {
    const uint64_t* p = reinterpret_cast<const uint64_t*>(partial);
    uint64_t acc = 0;
    for (int64_t i = begin + threadIdx.x; i < end; i += BLOCK) acc += p[i];
    s = static_cast<double>(block_sum(acc, s_u));
  } else {
    const double* p = reinterpret_cast<const double*>(partial);
    double acc = 0.0;
    for (int64_t i = begin + threadIdx.x; i < end; i += BLOCK) acc += p[i];
    s = block_sum(acc, s_d);
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
  hipLaunchKernelGGL(finalize_kernel, dim3(nrows + 1), dim3(BLOCK), 0, st,
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
  const int64_t by_device =
      std::max<int64_t>(1, static_cast<int64_t>(cu_count(device)) * PIX_WG_PER_CU / n_images);
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
  if (!a || !b || !partial) return FA_E_ARG;
  if (op < 0 || op > 3) return FA_E_OP;
  if (n_images <= 0 || n_per_image <= 0 || bpi <= 0) return FA_E_SHAPE;
  if (n_images > 65535 || static_cast<int64_t>(bpi) * BLOCK > INT32_MAX) return FA_E_SHAPE;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(bpi), static_cast<unsigned>(n_images));
  const uintptr_t rel = reinterpret_cast<uintptr_t>(a) - reinterpret_cast<uintptr_t>(b);

  bool exact = false;
  if (dtype == FA_U8) {
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
  return launch_finalize(partial, exact, static_cast<int>(n_images), bpi, n_each,
                         n_each * static_cast<double>(n_images), psnr_bias,
                         out_per_image, out_total, out_psnr_per_image,
                         out_psnr_total, st);
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
  v.bpi = bpi;
  v.param = param;
  v.partial = partial;
  // uint8 rows whose every start is 4-byte aligned are read as dwords
  const uintptr_t bases = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
  const int64_t strides = va[0] | va[1] | va[2] | vb[0] | vb[1] | vb[2];
  const bool dw = dtype == FA_U8 && !luma && W % 4 == 0 && (bases & 3) == 0 && (strides & 3) == 0;

  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(bpi), static_cast<unsigned>(n_images));
  const int rc = luma ? launch_view_dtype<true>(dtype, op, dw, grid, st, v)
                      : launch_view_dtype<false>(dtype, op, dw, grid, st, v);
  if (rc != FA_OK) return rc;
  const bool exact = dtype == FA_U8 && !luma && (op == FA_OP_MSE || op == FA_OP_L1);
  const double n_each = static_cast<double>(v.Cout) * plane;
  return launch_finalize(partial, exact, static_cast<int>(n_images), bpi, n_each,
                         n_each * static_cast<double>(n_images), psnr_bias, out_per_image,
                         out_total, out_psnr_per_image, out_psnr_total, st);
}

}  // extern "C"
