// SSIM forward over uint8 planes with both Gaussian passes on the matrix cores
// (v_mfma_f32_16x16x32_f16).  The same statistics as the strip engine's
// forward (fa_strip.h + SsimPol in fa_ssim.hip; reference: the fused SSIM
// kernel, fa_cuda.cu:389-637): the separable window over x', y', x'y' and
// (x' - y')^2 with x' = x - 128, then the SSIM formula per output pixel.
//
// Work split.  A wave owns a column strip of 16 output columns and walks down
// a chunk of output rows, 16 rows per step; a workgroup is four neighbouring
// strips.  There is no LDS traffic and no barrier until the final reduction.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (lane l, g = l / 16, n = l % 16):
//   A[m = n][k = 8g + i], B[k = 8g + i][n], D[m = 4g + i][n].
//
// Horizontal pass, one 16 x 16 block H_j per step:  H[r][c] = sum_k P[r][k] w(k - c)
//   A = the raw planes: lane l holds row n of the 16-row block, input columns
//       8g .. 8g+7 of the wave's 32-column window (one 8-byte load of x, one
//       of y), turned into exact fp16 operands:
//         x' and y' (integers in [-128, 127]),
//         x'y' = p3h + p3l and (x-y)^2 = p4h + p4l: the fp16 rounding of the
//         product (v_pk_mul_f16) and its remainder (v_pk_fma_f16 of the same
//         operands minus the rounded product, exact: an integer of at most
//         4 or 16 units),
//       built with v_perm_b32 and packed fp16 arithmetic on the bit patterns
//       0x64vv = 1024 + v, every plane scaled by 2^-9, all exactly.
//   B = the window scaled by 2^9 and split into fp16 hi + lo pieces (the scale
//       keeps the low piece of the smallest Gaussian weight normal).  The
//       scales cancel, products of fp16 operands are exact and accumulate in
//       float32: each H value carries the window to 22 bits, with float32
//       accumulation as in the vector-ALU kernel.  12 MFMAs per block.
//
// Vertical pass, 16 output rows from H_j and H_{j+1}:  O[r][c] = sum_k w(k - r) H[k][c]
//   B = the H values split into fp16 hi + lo; the D fragment of the
//       horizontal pass already holds rows 4g .. 4g+3 of its block in column
//       n, which is the B fragment's column n, so the rows of H_j and H_{j+1}
//       sit in k = 8g + i as (block j, rows 4g+i) for i < 4 and (block j+1,
//       rows 4g+i-4) for i >= 4.  The sum over k does not care about order,
//       so the A fragment (the window scaled by 2^9, hi + lo) is laid out to
//       match; even and odd steps swap which half of the B fragment holds the
//       newer block, and the A fragment's halves swap with it, so the H values
//       never move.  12 MFMAs per block (hi.hi, lo.hi, hi.lo per moment).
//   D = rows 4g .. 4g+3 of the output block in column n, scaled by 2^9: every
//       lane finishes four output pixels with all four moments in its own
//       registers.
#include "fa_ssim_mfma.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace fa {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <class To, class From>
__device__ inline To bc(From v) {
  return __builtin_bit_cast(To, v);
}

constexpr int MT = 16;                 // rows / columns of an MFMA block
constexpr float WSCALE = 512.0f;       // window scale of both passes (data: 2^-9)
constexpr int MF_MAX_K = 16;           // 16 output rows + K - 1 <= 32 input rows

// MF_CSO: the CS pass without the SSIM sums (the cs sums alone, which is all
// MS-SSIM reads below its coarsest scale).
enum { MF_REDUCE = 0, MF_MAP = 1, MF_CS = 2, MF_CSO = 3 };

// What the planes hold: uint8 samples, the float32 levels of a uint8 image's
// 2 x 2-mean pyramid (multiples of 4^-s in [0, 255], s <= 4), or its first
// level stored as float16 (multiples of 1/4 in [0, 255], exact in fp16).
enum { SRC_U8 = 0, SRC_F32 = 1, SRC_F16 = 2 };

// Buffer-resource word 3 for raw (untyped, unswizzled) access.
constexpr int MF_RSRC_WORD3 = 0x00020000;

struct MfArgs {
  const void* x;  // uint8 samples, or samples of a uint8 pyramid level (SRC_F32 / F16)
  const void* y;
  int64_t xsn, xsc, ysn, ysc;
  uint32_t xsh, ysh;
  int C, H, W, Hout, Wout, K;
  int TH, strips, tiles;
  int nbig, THs;   // a column's chunks: nbig of TH rows, then chunks of THs rows
  int xcd_planes;  // > 0: an XCD's range of tiles holds this many whole planes,
                   // walked chunk by chunk (every big chunk before any small one)
  const float* win;
  float C1, C2;
  float one;      // 1.0f (see split_pair)
  float* map;
  double* partial;
  double* partial_cs;   // MF_CS, MF_CSO
  void* px;             // MF_CS, MF_CSO: optional pyramid level (2 x 2 means),
  void* py;             //   float32, or float16 (level_f16, uint8 input)
  int level_f16;
  void* dpx[2];         // LVL_F32D: the two levels below px / py (float32, either
  void* dpy[2];         //   pair may be null)
  // the one-launch finish (ssim_mfma_kernel<..., FIN_SSIM>); FIN_MS uses acc
  // (this scale's words) and fscale
  uint64_t* acc;
  double fscale, finv, npix_img, npix_all;
  double *out_per_image, *out_total;
  int N;
};

// The one-launch finish of the uint8 forward (fa_gpu_ssim_once): the packed
// fixed-point words of ssim_fin_add (fa_common.h), which the strip kernel's
// finish shares.
constexpr int MF_COUNT_BITS = SSIM_FIN_COUNT_BITS;
constexpr int MF_STRIDE = SSIM_FIN_STRIDE;
constexpr int MF_FIN_MAX_IMAGES = SSIM_FIN_MAX_IMAGES;

__device__ inline void mf_finish(const MfArgs& a, int img, int wg_per_image, double s) {
  const SsimFin f = {a.acc, a.fscale, a.finv, a.npix_img, a.npix_all, a.N, a.out_per_image,
                     a.out_total};
  ssim_fin_add(f, img, wg_per_image, s);
}

// MS-SSIM's words: one per (scale, plane), each workgroup adding its sum of
// the plane's cs (or, at the coarsest scale, SSIM) values packed as mf_finish
// packs them, round(sum * 2^F) << MF_COUNT_BITS plus a count of 1, with
// F = 51 - bits(2 * output pixels of the plane at that scale).
__device__ inline uint64_t ms_add(uint64_t* w, double s, double fscale) {
  const int64_t f = __double2ll_rn(s * fscale);
  return __hip_atomic_fetch_add(w, (static_cast<uint64_t>(f) << MF_COUNT_BITS) + 1u,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline f4 mfma(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The six fp16 A fragments of one lane's 8 pixels of x and y: the planes
// x', y', and the hi + lo pieces of x'y' and (x' - y')^2, all scaled by 2^-9
// (exact: small integers times powers of two, and remainders that are
// multiples of 2^-9), so one set of weights serves all six.
struct Frag {
  h8 x, y, p3h, p3l, p4h, p4l;
  h8 xl, yl;  // pyramid levels only: the low fp16 pieces of x', y'
};

// The six fragments from eight samples of x and of y held as four fp16 pairs
// t = v + b, where the bias b is 1024 (uint8 bytes under the pattern 0x64vv)
// or 0 (float16 pyramid level, v a multiple of 1/4); cs = -(128 + b) 2^-9 and
// cu = -(128 + b) recentre them:
//   t 2^-9 + cs = (v - 128) 2^-9 = x' 2^-9,   t + cu = x'.
// Every value below is exact in fp16 for both sources (checked exhaustively
// over all pairs of sample values).
__device__ inline Frag prep_pairs(const h2 (&xt)[4], const h2 (&yt)[4], h2 cs, h2 cu) {
  u4 ox, oy, o3h, o3l, o4h, o4l;
  const h2 m = {static_cast<_Float16>(0x1p-9f), static_cast<_Float16>(0x1p-9f)};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const h2 xs = __builtin_elementwise_fma(xt[j], m, cs);  // x' 2^-9
    const h2 ys = __builtin_elementwise_fma(yt[j], m, cs);  // y' 2^-9
    const h2 xu = xt[j] + cu;                               // x'
    const h2 du = xt[j] - yt[j];                            // x' - y'
    const h2 ds = xs - ys;                                  // (x' - y') 2^-9
    // x'y' 2^-9 in [-31.75, 32] and (x'-y')^2 2^-9 in [0, 127]: the product
    // rounded to fp16, then the exact remainder from a fused multiply-add of
    // the same operands (at most 4, resp. 16, units of 2^-9 for bytes; a
    // multiple of 2^-13 of at most 2^-7, resp. 2^-5, for quarter samples)
    const h2 p3h = xu * ys;
    const h2 p3l = __builtin_elementwise_fma(xu, ys, -p3h);
    const h2 p4h = du * ds;
    const h2 p4l = __builtin_elementwise_fma(du, ds, -p4h);
    ox[j] = bc<uint32_t>(xs);
    oy[j] = bc<uint32_t>(ys);
    o3h[j] = bc<uint32_t>(p3h);
    o3l[j] = bc<uint32_t>(p3l);
    o4h[j] = bc<uint32_t>(p4h);
    o4l[j] = bc<uint32_t>(p4l);
  }
  Frag f;
  f.x = bc<h8>(ox);
  f.y = bc<h8>(oy);
  f.p3h = bc<h8>(o3h);
  f.p3l = bc<h8>(o3l);
  f.p4h = bc<h8>(o4h);
  f.p4l = bc<h8>(o4l);
  return f;
}

// uint8: v_perm_b32 places each byte under 0x64, the fp16 pattern of 1024 + v.
__device__ inline Frag prep(uint2 xa, uint2 ya) {
  h2 xt[4], yt[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t xw = j < 2 ? xa.x : xa.y;
    const uint32_t yw = j < 2 ? ya.x : ya.y;
    // v_perm_b32 picks bytes of {S0 : S1}: 0-3 from S1, 4-7 from S0
    const uint32_t sf = (j & 1) ? 0x04030402u : 0x04010400u;  // two bytes under 0x64
    xt[j] = bc<h2>(__builtin_amdgcn_perm(0x64646464u, xw, sf));
    yt[j] = bc<h2>(__builtin_amdgcn_perm(0x64646464u, yw, sf));
  }
  const h2 cs = {static_cast<_Float16>(-2.25f), static_cast<_Float16>(-2.25f)};
  const h2 cu = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  return prep_pairs(xt, yt, cs, cu);
}

// fp16 hi + lo of v (|v| < 65504): hi rounds to nearest, lo rounds the exact
// remainder, so hi + lo carries v to 2^-22.
__device__ inline void split2(float v, _Float16& hi, _Float16& lo) {
  hi = static_cast<_Float16>(v);
  lo = static_cast<_Float16>(v - static_cast<float>(hi));
}

// fp16 hi + lo of two values as packed pairs: hi is packed with one
// v_cvt_pkrtz (rounding toward zero), lo rounds the exact remainder, so
// hi + lo carries each value to 2^-21.  `one` is 1.0f from the kernel
// arguments: the remainder is written as fma(v, one, -hi), which the compiler
// cannot fold back to a subtraction, so it maps onto v_fma_mix (reading hi
// from the packed pair) instead of convert, subtract, convert.
__device__ inline void split_pair(float v0, float v1, float one, uint32_t& hi, uint32_t& lo) {
  const h2 h = bc<h2>(__builtin_amdgcn_cvt_pkrtz(v0, v1));
  const h2 l = {static_cast<_Float16>(__builtin_fmaf(v0, one, -static_cast<float>(h.x))),
                static_cast<_Float16>(__builtin_fmaf(v1, one, -static_cast<float>(h.y)))};
  hi = bc<uint32_t>(h);
  lo = bc<uint32_t>(l);
}

// The four H values of a D fragment into half HALF (u4 elements 2 HALF,
// 2 HALF + 1) of the vertical pass's B fragments.
template <int HALF, bool PYR>
__device__ inline void stash(f4 h, float one, u4& bhi, u4& blo) {
  // pyramid levels are not pre-scaled, so their sums carry the window's 2^9
  constexpr float sc = PYR ? 1.0f / WSCALE : 1.0f;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    uint32_t hi, lo;
    split_pair(h[2 * p] * sc, h[2 * p + 1] * sc, one, hi, lo);
    bhi[2 * HALF + p] = hi;
    blo[2 * HALF + p] = lo;
  }
}

struct Weights {
  h8 bh, bl;      // horizontal B: w(8g + i - n) * 2^9, hi and lo
  h8 eh, el;      // vertical A, even steps: block j in k = 8g + 0..3 (odd
                  // steps: halves swapped, block j in k = 8g + 4..7)
};

// The window, zero padded, in LDS: swin[16 + d] = w(d) for -16 <= d < 32
// (every tap offset a fragment uses).  Each wave fills its own copy, one
// load per lane, and reads it back in the same wave (LDS operations of a wave
// complete in order), so no barrier is needed and the 16 tap reads per lane
// are unconditional.
constexpr int WIN_PAD = 16, WIN_LEN = 48;

// Row pitch (floats) of the map's LDS staging: 64 columns and 4 of padding,
// which spreads a wave's writes (rows 4g + i, columns n) and its row reads
// over distinct banks.
constexpr int MAP_PITCH = 68;

__device__ inline void stage_window(const float* win, int K, float* sw, int lane) {
  if (lane < WIN_LEN) {
    const int d = lane - WIN_PAD;
    sw[lane] = (d >= 0 && d < K) ? win[d] : 0.0f;
  }
}

__device__ inline float tap(const float* sw, int d) { return sw[WIN_PAD + d]; }

__device__ inline Weights load_weights(const float* sw, int g, int n) {
  Weights w;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    _Float16 hi, lo;
    const float wh = tap(sw, 8 * g + i - n) * WSCALE;
    split2(wh, hi, lo);
    w.bh[i] = hi;
    w.bl[i] = lo;
    // input row (relative to the older block) that k = 8g + i stands for
    const int re = i < 4 ? 4 * g + i : MT + 4 * g + (i - 4);
    split2(tap(sw, re - n) * WSCALE, hi, lo);
    w.eh[i] = hi;
    w.el[i] = lo;
  }
  return w;
}

// The vertical pass's B fragments, per moment plane.
struct VState {
  u4 hi[4], lo[4];
};

// Horizontal sums of one 16-row block: E x', E y', E x'y', E (x'-y')^2
// along the row (the data's 2^-9 and the window's 2^9 cancel).
struct HAcc {
  f4 x, y, p3, p4;
};

// 12 MFMAs either way.  uint8: x', y' are exact single pieces (2 each), the
// byte pieces of x'y' and (x-y)^2 take both window pieces (4 each).  Pyramid
// levels: every plane is hi + lo and the lo.lo product (2^-22 of the sum) is
// left out (3 each).
template <bool PYR>
__device__ inline HAcc hmfma(const Frag& f, const Weights& w) {
  const f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  HAcc h;
  h.x = mfma(f.x, w.bh, z);
  h.y = mfma(f.y, w.bh, z);
  h.p3 = mfma(f.p3h, w.bh, z);
  h.p4 = mfma(f.p4h, w.bh, z);
  h.x = mfma(f.x, w.bl, h.x);
  h.y = mfma(f.y, w.bl, h.y);
  h.p3 = mfma(f.p3h, w.bl, h.p3);
  h.p4 = mfma(f.p4h, w.bl, h.p4);
  h.p3 = mfma(f.p3l, w.bh, h.p3);
  h.p4 = mfma(f.p4l, w.bh, h.p4);
  if constexpr (PYR) {
    h.x = mfma(f.xl, w.bh, h.x);
    h.y = mfma(f.yl, w.bh, h.y);
  } else {
    h.p3 = mfma(f.p3l, w.bl, h.p3);
    h.p4 = mfma(f.p4l, w.bl, h.p4);
  }
  return h;
}

template <int HALF, bool PYR>
__device__ inline void stash_all(const HAcc& h, float one, VState& v) {
  stash<HALF, PYR>(h.x, one, v.hi[0], v.lo[0]);
  stash<HALF, PYR>(h.y, one, v.hi[1], v.lo[1]);
  stash<HALF, PYR>(h.p3, one, v.hi[2], v.lo[2]);
  stash<HALF, PYR>(h.p4, one, v.hi[3], v.lo[3]);
}

// One lane's 8 samples of one 16-row block: 8 bytes of x and of y (uint8), 8
// floats of each (float32 pyramid levels) or 8 halves (float16 level).
template <int SRC>
struct Raw;
template <>
struct Raw<SRC_U8> {
  uint2 x, y;
};
template <>
struct Raw<SRC_F32> {
  float4 x0, x1, y0, y1;
};
template <>
struct Raw<SRC_F16> {
  u4 x, y;
};

__device__ inline Frag prep(const Raw<SRC_U8>& r, float) {
  return prep(r.x, r.y);
}

// The first level of a uint8 pyramid in float16: the samples are the fp16
// pairs themselves (bias 0).
__device__ inline Frag prep(const Raw<SRC_F16>& r, float) {
  h2 xt[4], yt[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    xt[j] = bc<h2>(r.x[j]);
    yt[j] = bc<h2>(r.y[j]);
  }
  const h2 cs = {static_cast<_Float16>(-0.25f), static_cast<_Float16>(-0.25f)};
  const h2 cu = {static_cast<_Float16>(-128.0f), static_cast<_Float16>(-128.0f)};
  return prep_pairs(xt, yt, cs, cu);
}

// Pyramid levels of uint8 input: every sample is a multiple of 4^-s in
// [0, 255] (s <= 4), so x' = x - 128 is exact in float32 and splits exactly
// into fp16 hi + lo (at most 16 significant bits); x'y' and (x'-y')^2 are
// formed in float32, as the strip kernel forms them, and split hi + lo (22
// bits).  No scaling: the window's 2^9 is taken out of the sums (stash).
__device__ inline Frag prep(const Raw<SRC_F32>& r, float one) {
  const float xs[8] = {r.x0.x, r.x0.y, r.x0.z, r.x0.w, r.x1.x, r.x1.y, r.x1.z, r.x1.w};
  const float ys[8] = {r.y0.x, r.y0.y, r.y0.z, r.y0.w, r.y1.x, r.y1.y, r.y1.z, r.y1.w};
  u4 ox, oxl, oy, oyl, o3h, o3l, o4h, o4l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a0 = xs[2 * j] - 128.0f, a1 = xs[2 * j + 1] - 128.0f;
    const float b0 = ys[2 * j] - 128.0f, b1 = ys[2 * j + 1] - 128.0f;
    const float d0 = a0 - b0, d1 = a1 - b1;
    uint32_t h, l;
    split_pair(a0, a1, one, h, l);
    ox[j] = h;
    oxl[j] = l;
    split_pair(b0, b1, one, h, l);
    oy[j] = h;
    oyl[j] = l;
    split_pair(a0 * b0, a1 * b1, one, h, l);
    o3h[j] = h;
    o3l[j] = l;
    split_pair(d0 * d0, d1 * d1, one, h, l);
    o4h[j] = h;
    o4l[j] = l;
  }
  Frag f;
  f.x = bc<h8>(ox);
  f.xl = bc<h8>(oxl);
  f.y = bc<h8>(oy);
  f.yl = bc<h8>(oyl);
  f.p3h = bc<h8>(o3h);
  f.p3l = bc<h8>(o3l);
  f.p4h = bc<h8>(o4h);
  f.p4l = bc<h8>(o4l);
  return f;
}

// Per-pixel SSIM from the four filtered moments, all scaled by 2^9:
//   U = 2^9 E x', V = 2^9 E y', X = 2^9 E x'y', Q = 2^9 E (x'-y')^2,
// with x' = x - 128 (any centre gives the same statistics):
//   A1 = 2 ux uy + 256 (ux + uy) + 2 * 128^2 + C1,  B1 = A1 + (ux - uy)^2
//   A2 = 2 (E x'y' - ux uy) + C2,  B2 = E (x'-y')^2 + A2 - (ux - uy)^2
struct Epi {
  float k1, C2;
  float k1s, c2s;  // 2^8 k1, 2^8 C2 (ssim_px_folded)
};

__device__ inline float ssim_px(const Epi& e, float U, float V, float X, float Q) {
  const float p = U * V;
  const float t = U + V;
  const float du = U - V;
  const float dd = du * 0x1p-18f;
  const float A1 = fmaf(0x1p-17f, p, fmaf(0.5f, t, e.k1));
  const float B1 = fmaf(dd, du, A1);
  const float A2 = fmaf(0x1p-8f, X, fmaf(-0x1p-17f, p, e.C2));
  const float B2 = fmaf(-dd, du, fmaf(0x1p-9f, Q, A2));
  return (A1 * A2) * __builtin_amdgcn_rcpf(B1 * B2);
}

// The same value with C2 folded into the vertical pass (the reduce kernel):
// the x'y' sums start at 2^8 C2, the first MFMA's accumulator input, so
// Xc = X + 2^8 C2, and A1, B1, A2, B2 are all taken times 2^8, which leaves
// the ratio unchanged:
//   A1' = 2^-9 U V + 2^7 (U + V) + 2^8 k1,  B1' = A1' + 2^-10 (U - V)^2
//   A2' = Xc - 2^-9 U V,                     B2' = A2' + Q / 2 - 2^-10 (U - V)^2
// One instruction fewer per pixel.  The map and CS kernels keep ssim_px:
// they have no registers to spare for the four-wide accumulator input.
__device__ inline float ssim_px_folded(const Epi& e, float U, float V, float Xc, float Q) {
  const float p = U * V;
  const float t = U + V;
  const float du = U - V;
  const float dd = du * 0x1p-10f;
  const float A1 = fmaf(0x1p-9f, p, fmaf(128.0f, t, e.k1s));
  const float B1 = fmaf(dd, du, A1);
  const float A2 = fmaf(-0x1p-9f, p, Xc);
  const float B2 = fmaf(-dd, du, fmaf(0.5f, Q, A2));
  return (A1 * A2) * __builtin_amdgcn_rcpf(B1 * B2);
}

// cs = A2 / B2 alone, with C2 folded into the vertical pass as in
// ssim_px_folded (A2' = Xc - 2^-9 U V, B2' = A2' + Q / 2 - 2^-10 (U - V)^2,
// both 2^8 times A2, B2): 8 instructions per pixel against 16 for the SSIM
// value and cs together.
__device__ inline float cs_px_folded(float U, float V, float Xc, float Q) {
  const float p = U * V;
  const float du = U - V;
  const float dd = du * 0x1p-10f;
  const float A2 = fmaf(-0x1p-9f, p, Xc);
  const float B2 = fmaf(-dd, du, fmaf(0.5f, Q, A2));
  return A2 * __builtin_amdgcn_rcpf(B2);
}

// cs = A2 / B2 beside the SSIM value (MS-SSIM's CS pass).
__device__ inline void ssim_cs_px(const Epi& e, float U, float V, float X, float Q, float& s,
                                  float& cs) {
  const float p = U * V;
  const float t = U + V;
  const float du = U - V;
  const float dd = du * 0x1p-18f;
  const float A1 = fmaf(0x1p-17f, p, fmaf(0.5f, t, e.k1));
  const float B1 = fmaf(dd, du, A1);
  const float A2 = fmaf(0x1p-8f, X, fmaf(-0x1p-17f, p, e.C2));
  const float B2 = fmaf(-dd, du, fmaf(0x1p-9f, Q, A2));
  // u = A2 / (B1 B2): ssim = A1 u, cs = B1 u
  const float u = A2 * __builtin_amdgcn_rcpf(B1 * B2);
  s = A1 * u;
  cs = B1 * u;
}

// Adds this lane's four outputs (rows row0 .. row0 + 3 of its column) to the
// lane's float64 sums (MF_CSO: the cs values into acc); `full` (uniform) says
// the whole 16 x 16 block lies inside the map.  MF_MAP also returns the four
// values in mv; the caller stores them (MF_MAP's stores in the kernel).
template <int MODE, bool FULL>
__device__ inline void finish(const Epi& e, const f4* o, int row0, int row_end, bool col_ok,
                              float (&mv)[4], double& acc, double& acc_cs) {
  float rs = 0.0f, rcs = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = FULL || (col_ok && row0 + i < row_end);
    if constexpr (MODE == MF_CS) {
      float s, cs;
      ssim_cs_px(e, o[0][i], o[1][i], o[2][i], o[3][i], s, cs);
      rs += ok ? s : 0.0f;
      rcs += ok ? cs : 0.0f;
    } else if constexpr (MODE == MF_CSO) {
      const float cs = cs_px_folded(o[0][i], o[1][i], o[2][i], o[3][i]);
      rs += ok ? cs : 0.0f;
    } else if constexpr (MODE == MF_MAP) {
      const float s = ssim_px(e, o[0][i], o[1][i], o[2][i], o[3][i]);
      mv[i] = s;  // stored by the caller, after the branch (see MapOut)
      rs += ok ? s : 0.0f;
    } else {
      const float s = ssim_px_folded(e, o[0][i], o[1][i], o[2][i], o[3][i]);
      rs += ok ? s : 0.0f;
    }
  }
  acc += static_cast<double>(rs);
  if constexpr (MODE == MF_CS) acc_cs += static_cast<double>(rcs);
}

// MS-SSIM's next pyramid level, as a matrix product of the A fragments the
// horizontal pass already holds: the 0/1 matrix P[k][c] = (k / 2 == c) sums
// column pairs of the 32-column window (B fragment: lane (g, n) holds
// P[8g + i][n]), and the D fragment holds, in lane (g, n), rows 4g .. 4g+3 of
// pooled column n, so each lane adds its two row pairs.  The sums are exact:
// four samples of x' 2^-9 (uint8, float16 level) or of x' = hi + lo (float32
// levels); the mean of four bytes, a multiple of 1/4, is exact in float16 too.
struct Pool {
  char* bx;        // this plane's level of x and y, at this chunk's first level row
  char* by;
  int rows;        // level rows this chunk writes (its input rows / 2)
  uint32_t rstep;  // bytes per level row
  uint32_t lo;     // this lane's byte offset in a block's level rows (row 2g,
                   // its column), or out of every buffer's range when it stores nothing
  h8 pm;           // the column-pair matrix fragment
  // LVL_F32D: the two levels below, as bx / by .. lo above (a block's 16 input
  // rows hold 4 rows of the first and 2 of the second)
  char *dx[2], *dy[2];
  int drows[2];
  uint32_t dstep[2], dlo[2];
};

// Lane exchanges of the deep levels' sums: v_mov_b32 with DPP quad_perm
// [1,0,3,2] / [2,3,0,1] (lanes n ^ 1, n ^ 2 in a row of 16) and a
// ds_swizzle in bit-mask mode with xor mask 16 (lane l ^ 16 in each half).
__device__ inline float lane_xor1(float v) {
  return bc<float>(__builtin_amdgcn_mov_dpp(bc<int>(v), 0xB1, 0xF, 0xF, false));
}
__device__ inline float lane_xor2(float v) {
  return bc<float>(__builtin_amdgcn_mov_dpp(bc<int>(v), 0x4E, 0xF, 0xF, false));
}
__device__ inline float lane_xor16(float v) {
  return bc<float>(__builtin_amdgcn_ds_swizzle(bc<int>(v), 0x401F));
}

// The 2 x 2 means of one block's level rows 2g and 2g + 1 (this lane's
// column), x and y: float32, or (HALF) float16 packed in pairs, which keeps
// them in two registers while they wait for the next block's loads.
template <bool HALF>
struct PoolOut {
  float mx[2], my[2];
};
template <>
struct PoolOut<true> {
  uint32_t hx, hy;  // rows 2g (low half) and 2g + 1 (high half)
};

template <bool PYR, bool HALF>
__device__ inline PoolOut<HALF> pool_frag(const Pool& pl, const Frag& f) {
  const f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 sx = mfma(f.x, pl.pm, z);
  f4 sy = mfma(f.y, pl.pm, z);
  if constexpr (PYR) {
    sx = mfma(f.xl, pl.pm, sx);
    sy = mfma(f.yl, pl.pm, sy);
  }
  // a sum of four is (S - 512) 2^-9 (uint8, float16 level) or S - 512: the
  // mean S / 4 is sum * k + 128
  constexpr float k = PYR ? 0.25f : 128.0f;
  float mx[2], my[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    mx[q] = fmaf(sx[2 * q] + sx[2 * q + 1], k, 128.0f);
    my[q] = fmaf(sy[2 * q] + sy[2 * q + 1], k, 128.0f);
  }
  PoolOut<HALF> po;
  if constexpr (HALF) {
    // exact: multiples of 1/4 in [0, 255]
    po.hx = bc<uint32_t>(h2{static_cast<_Float16>(mx[0]), static_cast<_Float16>(mx[1])});
    po.hy = bc<uint32_t>(h2{static_cast<_Float16>(my[0]), static_cast<_Float16>(my[1])});
  } else {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      po.mx[q] = mx[q];
      po.my[q] = my[q];
    }
  }
  return po;
}

// Stores block j's means through buffer resources whose base is the block's
// first level row (scalar) and whose range ends at the last row this chunk
// writes: the lane's offset is fixed, so a store costs no vector address
// arithmetic, and the range check drops the rows past the chunk and the lanes
// that store nothing.  Four stores in every block.
template <bool HALF>
__device__ inline void pool_store(const Pool& pl, int j, const PoolOut<HALF>& po) {
  const int row = MT / 2 * j;  // the block's first level row, in this chunk
  const uint32_t boff = static_cast<uint32_t>(row) * pl.rstep;
  const int range = max(pl.rows - row, 0) * static_cast<int>(pl.rstep);
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(pl.bx + boff, 0, range, MF_RSRC_WORD3);
  const auto ry = __builtin_amdgcn_make_buffer_rsrc(pl.by + boff, 0, range, MF_RSRC_WORD3);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int o = static_cast<int>(pl.lo + q * pl.rstep);  // level row 2g + q
    if constexpr (HALF) {
      const int sh = 16 * q;
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(po.hx >> sh), rx, o, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(po.hy >> sh), ry, o, 0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(bc<uint32_t>(po.mx[q]), rx, o, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(bc<uint32_t>(po.my[q]), ry, o, 0, 0);
    }
  }
}

// LVL_F32D: the two levels below a float32 level from the same block's
// means.  Lane (g, n) holds the level's rows 2g, 2g + 1 in column n; the sum
// of both rows over lanes n, n ^ 1 is 4 means of the next level down (its row
// g, column n / 2), and over the quad of lanes and g, g ^ 1 it is 16 means of
// the one below (row g / 2, column n / 4).  Every sum is exact: multiples of
// 1/16 below 2^12.  Stored like pool_store: four stores in every block.
__device__ inline void pool_store_deep(const Pool& pl, int j, const PoolOut<false>& po) {
  const float tx = po.mx[0] + po.mx[1], ty = po.my[0] + po.my[1];
  const float px = tx + lane_xor1(tx), py = ty + lane_xor1(ty);
  const float qx = px + lane_xor2(px), qy = py + lane_xor2(py);
  const float rx = qx + lane_xor16(qx), ry = qy + lane_xor16(qy);
  const float vx[2] = {px * 0.25f, rx * 0.0625f};
  const float vy[2] = {py * 0.25f, ry * 0.0625f};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const int row = (MT / 4 >> d) * j;  // the block's first row of that level, in this chunk
    const uint32_t boff = static_cast<uint32_t>(row) * pl.dstep[d];
    const int range = max(pl.drows[d] - row, 0) * static_cast<int>(pl.dstep[d]);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc(pl.dx[d] + boff, 0, range, MF_RSRC_WORD3);
    const auto ry = __builtin_amdgcn_make_buffer_rsrc(pl.dy[d] + boff, 0, range, MF_RSRC_WORD3);
    __builtin_amdgcn_raw_buffer_store_b32(bc<uint32_t>(vx[d]), rx, static_cast<int>(pl.dlo[d]), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(bc<uint32_t>(vy[d]), ry, static_cast<int>(pl.dlo[d]), 0, 0);
  }
}

// FOLD: the x'y' sums start at c2s (ssim_px_folded).
template <int PAR, bool FOLD>
__device__ inline void vblock(const Weights& w, const VState& v, f4* o, float c2s) {
  const f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  const f4 zc = {c2s, c2s, c2s, c2s};
  h8 ah = w.eh, al = w.el;
  if constexpr (PAR == 1) {
    // the odd layout is the even one with its halves swapped, built here in
    // each odd step (4 moves) so that it holds no registers between steps:
    // that keeps the REDUCE and MAP kernels within 128 VGPRs (4 waves/SIMD)
    u4 h = bc<u4>(w.eh), l = bc<u4>(w.el);
    asm volatile("" : "+v"(h), "+v"(l));  // keeps the copy inside the loop
    ah = bc<h8>(u4{h[2], h[3], h[0], h[1]});
    al = bc<h8>(u4{l[2], l[3], l[0], l[1]});
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = mfma(ah, bc<h8>(v.hi[q]), FOLD && q == 2 ? zc : z);
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = mfma(al, bc<h8>(v.hi[q]), o[q]);
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = mfma(ah, bc<h8>(v.lo[q]), o[q]);
}

// What a CS pass writes besides its sums: no level, the next pyramid level in
// float32, or in float16 (uint8 input only).
// LVL_F32D: the float32 level and the two below it (the float16 level's
// pass of a uint8 pyramid, so that the coarser scales can run side by side).
enum { LVL_NONE = 0, LVL_F32 = 1, LVL_F16 = 2, LVL_F32D = 3 };

// One workgroup's tile t of a launch over the planes of `a`: its 16-row
// blocks, walked down its chunk of its column strip by the four waves, each
// lane's sums added to acc (and acc_cs, MF_CS).  The tile's plane and its
// index within the plane come back for the caller's reduction.
template <int SRC, int MODE, int LVL>
__device__ __attribute__((always_inline)) inline void mf_walk(
    const MfArgs& a, int t, float (&swin)[WAVES_PER_BLOCK][WIN_LEN], double& acc,
    double& acc_cs, int& plane_out, int& tile_out, float* smap = nullptr) {
  constexpr bool PYR = SRC == SRC_F32;  // float32 samples: hi + lo operands
  constexpr bool LEVEL = LVL != LVL_NONE;
  static_assert(!LEVEL || MODE == MF_CS || MODE == MF_CSO, "levels come from the CS pass");
  static_assert(LVL != LVL_F16 || SRC == SRC_U8, "float16 levels below uint8 input only");
  static_assert(LVL != LVL_F32D || SRC == SRC_F16, "deep levels: the float16 level's pass");
  int plane, chunk, strip;
  if (a.xcd_planes > 0) {
    const int per = a.xcd_planes * a.tiles;  // the tiles of one XCD (xcd_tile)
    const int xr = t / per;
    const int i = t - xr * per;
    const int cols = a.xcd_planes * a.strips;
    chunk = i / cols;
    const int j = i - chunk * cols;
    plane = xr * a.xcd_planes + j / a.strips;
    strip = j - (j / a.strips) * a.strips;
  } else {
    plane = t / a.tiles;
    const int tl = t - plane * a.tiles;
    chunk = tl / a.strips;
    strip = tl - chunk * a.strips;
  }
  const int tile = chunk * a.strips + strip;
  // uniform (a scalar register): every branch on the wave's columns is a
  // scalar branch, so each path issues the same loads and stores
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
  const int lane = static_cast<int>(threadIdx.x) % WAVE;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int c0 = (strip * WAVES_PER_BLOCK + wave) * MT;  // first output column of the wave
  const int r0 = chunk < a.nbig ? chunk * a.TH : a.nbig * a.TH + (chunk - a.nbig) * a.THs;
  const int r_lim = r0 + (chunk < a.nbig ? a.TH : a.THs);  // the chunk's end row
  const int r_end = min(r_lim, a.Hout);
  plane_out = plane;
  tile_out = tile;

  // uniform per wave; the map kernel runs every wave of the workgroup (their
  // steps meet at a barrier, see the map's stores), a wave past the map with
  // its loads clamped into the image and its outputs masked
  if (MODE == MF_MAP || c0 < a.Wout) {
    const int img = plane / a.C;
    const int ch = plane - img * a.C;
    // element pointers of this plane (uint8 samples, or pyramid samples)
    using E = typename std::conditional<
        PYR, float, typename std::conditional<SRC == SRC_F16, _Float16, uint8_t>::type>::type;
    constexpr int EB = static_cast<int>(sizeof(E));  // bytes per sample
    const E* __restrict__ xp = reinterpret_cast<const E*>(a.x) + img * a.xsn + ch * a.xsc;
    const E* __restrict__ yp = reinterpret_cast<const E*>(a.y) + img * a.ysn + ch * a.ysc;
    // this lane's 8 input columns; a chunk past the image only feeds output
    // columns past Wout, so it is clamped (W % 8 == 0: chunks never straddle)
    const uint32_t cc = static_cast<uint32_t>(min(c0 + 8 * g, a.W - 8));
    stage_window(a.win, a.K, swin[wave], lane);
    const Weights w = load_weights(swin[wave], g, n);
    const float k1 = 2.0f * 128.0f * 128.0f + a.C1;
    const Epi e = {k1, a.C2, 256.0f * k1, 256.0f * a.C2};
    const bool col_ok = c0 + n < a.Wout;
    // MF_MAP: the plane's map, and the lane's column in its workgroup's 64
    // (0x80000000, past every range, where that lies outside the map; the host
    // keeps a plane's map below 2^31 bytes)
    float* const map_plane =
        MODE == MF_MAP ? a.map + static_cast<int64_t>(plane) * a.Hout * a.Wout : nullptr;
    const uint32_t map_row = static_cast<uint32_t>(a.Wout) * 4u;
    const int wg_col = strip * WAVES_PER_BLOCK * MT + lane;
    const uint32_t wg_col_off =
        wg_col < a.Wout ? static_cast<uint32_t>(wg_col) * 4u : 0x80000000u;

    // The pyramid level: a wave's 32-column window pools to 16 columns, its
    // own 8 (c0/2 .. c0/2 + 7) and its right neighbour's 8.  Even waves store
    // all 16 (64 contiguous bytes per level row), odd waves none; the last
    // active wave of a row, even or odd, stores its 16 up to the image edge,
    // which covers the columns of the waves past Wout (W <= c0 + 16 + K - 1
    // there).  Rows: this chunk's TH input rows, and in the last chunk
    // everything up to 2 floor(H / 2).  Every row the chunk pools lies in one
    // of its H blocks.
    Pool pl = {};
    if constexpr (LEVEL) {
      {
        const int Wd = a.W / 2;
        const int eb = LVL == LVL_F16 ? 2 : 4;
        const int row_end = r_lim >= a.Hout ? 2 * (a.H / 2) : r_lim;
        const int64_t first = (static_cast<int64_t>(plane) * (a.H / 2) + r0 / 2) * Wd * eb;
        pl.bx = static_cast<char*>(a.px) + first;
        pl.by = static_cast<char*>(a.py) + first;
        pl.rows = row_end / 2 - r0 / 2;
        pl.rstep = static_cast<uint32_t>(Wd * eb);
        const bool last_wave = c0 + MT >= a.Wout;
        const bool wave_on = (wave & 1) == 0 || last_wave;
        const bool lane_on = wave_on && c0 / 2 + n < Wd;
        // 0x80000000 lies past every range (a plane's level is below 2^31 bytes)
        pl.lo = lane_on ? static_cast<uint32_t>((2 * g * Wd + c0 / 2 + n) * eb) : 0x80000000u;
        if constexpr (LVL == LVL_F32D) {
          // level d + 2 below the input (d = 0, 1): W / 2^(d+2) columns (W % 8
          // == 0), floor(H / 2^(d+2)) rows; this chunk's rows r0 / 2^(d+2) ..;
          // lane (g, n) stores row g >> d, column (c0 / 2 + n) >> (d + 1)
          // when n (and, d = 1, g) is the first of its group
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const int sh = d + 2;
            const int Wl = a.W >> sh;
            const int end = r_lim >= a.Hout ? (a.H >> sh) : (r_lim >> sh);
            const bool have = a.dpx[d] != nullptr;
            const int64_t at = (static_cast<int64_t>(plane) * (a.H >> sh) + (r0 >> sh)) * Wl * 4;
            pl.dx[d] = static_cast<char*>(have ? a.dpx[d] : a.px) + (have ? at : 0);
            pl.dy[d] = static_cast<char*>(have ? a.dpy[d] : a.py) + (have ? at : 0);
            pl.drows[d] = have ? end - (r0 >> sh) : 0;
            pl.dstep[d] = static_cast<uint32_t>(Wl * 4);
            const int col = (c0 / 2 + n) >> (d + 1);
            const bool first = (n & ((2 << d) - 1)) == 0 && (d == 0 || (g & 1) == 0);
            pl.dlo[d] = wave_on && first && col < Wl
                            ? static_cast<uint32_t>(((g >> d) * Wl + col) * 4)
                            : 0x80000000u;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        pl.pm[i] = static_cast<_Float16>(((8 * g + i) >> 1) == n ? 1.0f : 0.0f);
    }

    // Rows past the image only feed output rows past Hout.  load(j) is called
    // for j = 0, 1, 2, ... in order, so the row offsets advance by 16 rows per
    // call.  uint8 blocks (and float16 levels) are read through a buffer
    // resource that starts at the block's first row and ends at the plane's
    // end: its base and range are scalar values, the lane's offset within the
    // block is fixed, so a load costs no vector instruction, and the range
    // check turns rows past the image into zeros without touching memory.
    // float32 levels clamp their offsets to the last row.
    const uint32_t xstep = MT * a.xsh, ystep = MT * a.ysh;
    const uint32_t rl = static_cast<uint32_t>(min(r0 + n, a.H - 1));
    const uint32_t xmax = static_cast<uint32_t>(a.H - 1) * a.xsh + cc;
    const uint32_t ymax = static_cast<uint32_t>(a.H - 1) * a.ysh + cc;
    uint32_t xo = rl * a.xsh + cc, yo = rl * a.ysh + cc;  // block 0
    // byte offsets within the block
    const uint32_t vx = (static_cast<uint32_t>(n) * a.xsh + cc) * EB;
    const uint32_t vy = (static_cast<uint32_t>(n) * a.ysh + cc) * EB;
    // plane samples and the block's first sample; the host keeps (H + 48) rows
    // of either plane below 2^31 bytes
    const int ext_x = (a.H - 1) * static_cast<int>(a.xsh) + a.W;
    const int ext_y = (a.H - 1) * static_cast<int>(a.ysh) + a.W;
    int bx = r0 * static_cast<int>(a.xsh), by = r0 * static_cast<int>(a.ysh);
    const int nb = (r_end - r0 + MT - 1) / MT;  // output blocks; H blocks 0 .. nb
    // Every step issues its load, whether or not its block is used, so that
    // every path through the loop issues the same memory operations (the
    // compiler then waits for the loads alone, see MapOut); a block past nb
    // gets an empty range (uint8, float16: nothing is read) or re-reads the
    // clamped last row (float32 levels).
    auto load = [&](int j, Raw<SRC>& r) {
      if constexpr (PYR) {
        r.x0 = *reinterpret_cast<const float4*>(xp + xo);
        r.x1 = *reinterpret_cast<const float4*>(xp + xo + 4);
        r.y0 = *reinterpret_cast<const float4*>(yp + yo);
        r.y1 = *reinterpret_cast<const float4*>(yp + yo + 4);
        xo = min(xo + xstep, xmax);
        yo = min(yo + ystep, ymax);
      } else {
        const bool live = j <= nb;  // uniform
        const auto rx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<E*>(xp + bx), 0, live ? max(ext_x - bx, 0) * EB : 0, MF_RSRC_WORD3);
        const auto ry = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<E*>(yp + by), 0, live ? max(ext_y - by, 0) * EB : 0, MF_RSRC_WORD3);
        if constexpr (SRC == SRC_F16) {
          r.x = bc<u4>(__builtin_amdgcn_raw_buffer_load_b128(rx, vx, 0, 0));
          r.y = bc<u4>(__builtin_amdgcn_raw_buffer_load_b128(ry, vy, 0, 0));
        } else {
          const auto lx = __builtin_amdgcn_raw_buffer_load_b64(rx, vx, 0, 0);
          const auto ly = __builtin_amdgcn_raw_buffer_load_b64(ry, vy, 0, 0);
          r.x = uint2{lx[0], lx[1]};
          r.y = uint2{ly[0], ly[1]};
        }
        bx += static_cast<int>(xstep);
        by += static_cast<int>(ystep);
      }
    };
    // horizontal pass of block j, and (LEVEL) its share of the pyramid, which
    // the caller stores after issuing the next block's loads (pool_store)
    // LATE: the level of block j waits in registers for the next block's
    // loads and is stored after them.  The uint8 cs-only pass with a float32
    // level has no four registers to spare (it would spill) and stores it
    // inside hpass, before those loads.
    constexpr bool HALF = LVL == LVL_F16;
    constexpr bool LATE = LEVEL && !(SRC == SRC_U8 && MODE == MF_CSO && LVL == LVL_F32);
    // GUARD: a step past the last block skips its loads and stores along
    // with its horizontal pass.  Both forms give the compiler the same
    // memory operations behind every wait (it waits with vmcnt(4) where a
    // step stores); they differ in the registers the compiler ends up with:
    // the guarded form keeps the uint8 kernels within 128 without spills,
    // the unguarded one the float16 and float32 level kernels.
    constexpr bool GUARD = SRC == SRC_U8;
    PoolOut<HALF> po = {};
    auto hpass = [&](int j, const Raw<SRC>& r) {
      const Frag f = prep(r, a.one);
      if constexpr (LEVEL) {
        po = pool_frag<PYR, HALF>(pl, f);
        if constexpr (!LATE) pool_store<HALF>(pl, j, po);
      }
      return hmfma<PYR>(f, w);
    };
    auto level_store = [&](int j) {
      if constexpr (LATE) pool_store<HALF>(pl, j, po);
      if constexpr (LVL == LVL_F32D) pool_store_deep(pl, j, po);
    };
    auto epilogue = [&](int b, const f4* o) {
      const int row0 = r0 + MT * b + 4 * g;
      float mv[4];
      if (r0 + MT * (b + 1) <= r_end && c0 + MT <= a.Wout)  // uniform: the whole block
        finish<MODE, true>(e, o, row0, r_end, col_ok, mv, acc, acc_cs);
      else
        finish<MODE, false>(e, o, row0, r_end, col_ok, mv, acc, acc_cs);
      if constexpr (MODE == MF_MAP) {
        // MF_MAP's stores.  A lane holds rows 4g .. 4g+3 of one column, so
        // stored straight from the fragment each store instruction covers 64
        // bytes of four rows, most pieces split over two 128-byte lines (map
        // rows of 7640 bytes at configs[1]); the texture units then spent ~51
        // cycles per store and were 83 % busy.  Instead the four waves stage
        // the workgroup's 16 x 64 block in LDS (rows padded to 68 floats:
        // conflict-free both ways, double-buffered so one barrier per step
        // suffices) and each wave stores four whole rows, 256 contiguous
        // bytes per instruction.  The barrier waits for LDS only: a fence
        // there would wait for the next block's loads in flight.  The stores
        // go through a buffer resource whose base is the block's first map row
        // (scalar) and whose range ends at the chunk's last row, so the range
        // check drops the rows past the chunk (and the 0x80000000 offsets the
        // columns past the map); they are issued on every path, so the
        // compiler waits for the next block's loads alone (vmcnt(4)).
        const int rb = r0 + MT * b;
        const auto r = __builtin_amdgcn_make_buffer_rsrc(
            map_plane + static_cast<int64_t>(rb) * a.Wout, 0,
            max(r_end - rb, 0) * static_cast<int>(map_row), MF_RSRC_WORD3);
        float* stg = smap + (b & 1) * (MT * MAP_PITCH);
#pragma unroll
        for (int i = 0; i < 4; ++i) stg[(4 * g + i) * MAP_PITCH + MT * wave + n] = mv[i];
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int row = 4 * wave + k;
          __builtin_amdgcn_raw_buffer_store_b32(bc<uint32_t>(stg[row * MAP_PITCH + lane]), r,
                                                static_cast<uint32_t>(row) * map_row + wg_col_off,
                                                0, 0);
        }
      }
    };

    // Software pipeline: the horizontal MFMAs of block j + 2 are issued
    // between the vertical MFMAs of step j and its epilogue, so the matrix
    // cores and the vector ALU overlap within the wave too.
    //
    // Memory order per step: the wait for block j's loads (in hpass), the
    // loads of block j + 1, then the step's stores (the level of block j,
    // the map of the step's output block).  The stores are unconditional
    // (the range checks drop what lies past the chunk), so on every path into
    // the next step's wait four stores follow the loads it waits for, and the
    // compiler waits with vmcnt(4): the stores stay in flight.  The first
    // step (peeled) is the only one whose loads may have nothing behind them.
    VState v;
    Raw<SRC> raw;
    load(0, raw);
    stash_all<0, PYR>(hpass(0, raw), a.one, v);
    load(1, raw);
    level_store(0);
    HAcc hn = hpass(1, raw);
    load(2, raw);
    level_store(1);
    // step with output block b: PAR 0 finds H_b in the first half of the
    // vertical operand and puts H_{b+1} in the second, PAR 1 the reverse
    auto step = [&](int b, auto par) {
      constexpr int PAR = decltype(par)::value;
      stash_all<1 - PAR, PYR>(hn, a.one, v);  // H_{b+1} into the half H_{b-1} held
      f4 o[4];
      vblock<PAR, MODE == MF_REDUCE || MODE == MF_CSO>(w, v, o, e.c2s);
      if constexpr (GUARD) {
        if (b + 2 <= nb) {  // uniform
          hn = hpass(b + 2, raw);
          load(b + 3, raw);
          level_store(b + 2);
        }
      } else {
        if (b + 2 <= nb) hn = hpass(b + 2, raw);  // uniform
        load(b + 3, raw);
        level_store(b + 2);
      }
      epilogue(b, o);
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    step(0, P0{});  // nb >= 1; with nb == 0 its sums and stores would be dropped
    for (int b = 1; b < nb; b += 2) {
      step(b, P1{});
      if (b + 1 >= nb) break;
      step(b + 1, P0{});
    }
  }
}

// What a launch does with its workgroups' sums: store them as partial slots
// (FIN_NONE), finish the uint8 forward's means (FIN_SSIM, mf_finish), or add
// them to MS-SSIM's per-(scale, plane) words (FIN_MS, ms_add).
enum { FIN_NONE = 0, FIN_SSIM = 1, FIN_MS = 2 };

// uint8 and float16 levels: 4 waves per SIMD (128 VGPRs) fit without spills
// and beat 3; the uint8 cs-only pass writing a float32 level (which MS-SSIM
// does not use: its first level is float16) needs more and runs 3, and so
// does the float16 level's pass writing three levels (which spills at 128;
// at 1080p its 720 workgroups fit 3 per CU anyway).  LVL (CS modes): the
// pyramid level the pass writes.
template <int SRC, int MODE, int LVL, int FIN = FIN_NONE>
__global__ __launch_bounds__(BLOCK)
__attribute__((amdgpu_waves_per_eu(
    SRC == SRC_F32 ? 1
    : ((SRC == SRC_U8 && MODE == MF_CSO && LVL == LVL_F32) || LVL == LVL_F32D) ? 3
                                                                             : 4)))
void ssim_mfma_kernel(MfArgs a) {
  static_assert(FIN != FIN_SSIM || (MODE == MF_REDUCE && SRC == SRC_U8),
                "the finish: uint8 forward sums");
  static_assert(FIN != FIN_MS || MODE == MF_CSO, "MS-SSIM's words: the cs sums of a scale");
  __shared__ double sred[2 * WAVES_PER_BLOCK];
  __shared__ float swin[WAVES_PER_BLOCK][WIN_LEN];
  __shared__ float smap[MODE == MF_MAP ? 2 * MT * MAP_PITCH : 1];  // the map's staging
  double acc = 0.0, acc_cs = 0.0;
  int plane = 0, tile = 0;
  mf_walk<SRC, MODE, LVL>(a, static_cast<int>(xcd_tile(blockIdx.x, gridDim.x)), swin, acc,
                          acc_cs, plane, tile, smap);
  // packed: each image owns C * tiles consecutive slots, as the finalize reads them
  const int64_t slot = static_cast<int64_t>(plane) * a.tiles + tile;
  if constexpr (MODE == MF_CS) {
    double s = 0.0, scs = 0.0;
    block_sum2(acc, acc_cs, sred, &s, &scs);
    if (threadIdx.x == 0) {
      a.partial[slot] = s;
      a.partial_cs[slot] = scs;
    }
  } else {
    const double s = block_sum(acc, sred);
    if constexpr (FIN == FIN_SSIM) {
      if (threadIdx.x == 0) mf_finish(a, plane / a.C, a.C * a.tiles, s);
    } else if constexpr (FIN == FIN_MS) {
      if (threadIdx.x == 0) ms_add(a.acc + static_cast<int64_t>(plane) * MF_STRIDE, s, a.fscale);
    } else if (threadIdx.x == 0) {
      (MODE == MF_CSO ? a.partial_cs : a.partial)[slot] = s;
    }
  }
}

// MS-SSIM's coarse scales (2 .. M - 1 of a uint8 pyramid, float32 levels) in
// one launch, and the reduction of every scale after them.  The scales'
// workgroups follow each other in the grid (coarser last, so their short
// tiles fill the end of the launch); each adds its cs sum (the coarsest
// scale: its SSIM sum) to its (scale, plane) word with a returning atomic.
// The workgroup whose add completes a word's count (the scale's tiles per
// plane) adds 1 to the launch's counter; the one that completes the counter
// holds the only view in which every word is whole -- the scales before this
// launch added theirs in earlier launches on the stream -- and turns them into
// the result: each plane's means, clamped at zero and raised to the scale's
// weight, multiplied over the scales (reference functional.py:897-901), the
// channel mean of each image and the mean over the batch, as ms_term_kernel and
// ms_finish_kernel do from partial sums.  It reads the words with atomic
// exchanges of zero and resets the counter, so the accumulator is zero again
// for the next call.  A returning atomic has been performed where every agent
// sees it once its value is back, so a count that completes has every add of
// that word behind it.
constexpr int MS_TAIL_MAX = 3;         // scales 2 .. 4 of a five-scale pyramid
constexpr int MS_WORD_SCALES = 8;
constexpr int MS_FIN_MAX_PLANES = 256;
static_assert(FA_MS_SSIM_ACC_WORDS == (MS_WORD_SCALES * MS_FIN_MAX_PLANES + 1) * MF_STRIDE,
              "the ABI's accumulator size");

struct MfTail {
  MfArgs s[MS_TAIL_MAX];
  int n, first;                 // scales first .. first + n - 1 in this launch
  int wg_end[MS_TAIL_MAX];      // end of each scale's workgroups in the grid
  int M, N, C, planes;
  uint64_t* words;              // word (m, plane) at (m * planes + plane) * MF_STRIDE,
                                // the launch's counter after M * planes of them
  double finv[MS_WORD_SCALES];  // 2^-F of every scale's words
  double npix[MS_WORD_SCALES];  // output pixels of a plane at each scale
  double w[MS_WORD_SCALES];     // the scales' exponents
  double *out_per_image, *out_total;
};

__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(1)))
void ssim_mfma_tail_kernel(MfTail m) {
  __shared__ double sred[2 * WAVES_PER_BLOCK];
  __shared__ float swin[WAVES_PER_BLOCK][WIN_LEN];
  __shared__ double sterm[(2 + MS_TAIL_MAX) * MS_FIN_MAX_PLANES];
  __shared__ int sfin;
  const int b = static_cast<int>(blockIdx.x);
  int k = 0;
  while (k + 1 < m.n && b >= m.wg_end[k]) ++k;
  k = __builtin_amdgcn_readfirstlane(k);
  const MfArgs& a = m.s[k];
  double acc = 0.0, acc_cs = 0.0;
  int plane = 0, tile = 0;
  // the coarsest scale's SSIM values, the cs values of the others, with the
  // per-pixel arithmetic of the per-scale passes (MF_CS there, MF_CSO's folded
  // form here); either way the sum the word takes ends up in acc
  const int t = b - (k > 0 ? m.wg_end[k - 1] : 0);
  if (k == m.n - 1)
    mf_walk<SRC_F32, MF_CS, LVL_NONE>(a, t, swin, acc, acc_cs, plane, tile);
  else
    mf_walk<SRC_F32, MF_CSO, LVL_NONE>(a, t, swin, acc, acc_cs, plane, tile);
  const double s = block_sum(acc, sred);
  const int64_t planes = m.planes;
  if (threadIdx.x == 0) {
    constexpr uint64_t CM = (uint64_t(1) << MF_COUNT_BITS) - 1;
    const int64_t sc = m.first + k;
    const uint64_t old = ms_add(m.words + (sc * planes + plane) * MF_STRIDE, s, a.fscale);
    int fin = 0;
    if ((old & CM) + 1u == static_cast<uint64_t>(a.tiles)) {
      uint64_t* cnt = m.words + static_cast<int64_t>(m.M) * planes * MF_STRIDE;
      const uint64_t c = __hip_atomic_fetch_add(cnt, uint64_t(1), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      if (c + 1u == static_cast<uint64_t>(m.n) * planes) {
        __hip_atomic_store(cnt, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        fin = 1;
      }
    }
    sfin = fin;
  }
  __syncthreads();
  if (!sfin) return;
  // one word per thread (every exchange of the workgroup in flight at once):
  // word i is scale i / planes, plane i % planes; its term into sterm[i]
  const int64_t words = static_cast<int64_t>(m.M) * planes;
  for (int64_t i = threadIdx.x; i < words; i += BLOCK) {
    const int sc = static_cast<int>(i / planes);
    const uint64_t v = __hip_atomic_exchange(m.words + i * MF_STRIDE, uint64_t(0),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const double mean =
        static_cast<double>(static_cast<int64_t>(v) >> MF_COUNT_BITS) * m.finv[sc] / m.npix[sc];
    sterm[i] = pow(mean > 0.0 ? mean : 0.0, m.w[sc]);
  }
  __syncthreads();
  // each plane's product over the scales, in scale order, into sterm[plane]
  for (int64_t p = threadIdx.x; p < planes; p += BLOCK) {
    double prod = 1.0;
    for (int sc = 0; sc < m.M; ++sc) prod *= sterm[sc * planes + p];
    sterm[p] = prod;
  }
  __syncthreads();
  double tot = 0.0;
  for (int n = threadIdx.x; n < m.N; n += BLOCK) {
    double img = 0.0;
    for (int c = 0; c < m.C; ++c) img += sterm[n * m.C + c];
    img /= static_cast<double>(m.C);
    if (m.out_per_image) m.out_per_image[n] = img;
    tot += img;
  }
  tot = block_sum(tot, sred);
  if (threadIdx.x == 0 && m.out_total) *m.out_total = tot / static_cast<double>(m.N);
}

// FA_SSIM_MFMA=0 in the environment selects the vector-ALU kernel instead.
bool mfma_enabled() {
  const char* e = std::getenv("FA_SSIM_MFMA");
  return !(e && e[0] == '0');
}

template <int SRC, int MODE, int LVL, int FIN = FIN_NONE>
int occupancy() {
  static int occ = 0;
  if (occ <= 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &v, reinterpret_cast<const void*>(&ssim_mfma_kernel<SRC, MODE, LVL, FIN>), BLOCK,
            0) != hipSuccess ||
        v <= 0)
      v = 1;
    occ = v;
  }
  return occ;
}

// The kernel of (source, mode, level): its occupancy (launch == false) or its
// launch.
template <int SRC, int MODE, int LVL>
int run(bool launch, dim3 grid, hipStream_t st, const MfArgs& a) {
  if constexpr (SRC == SRC_U8 && MODE == MF_REDUCE) {
    if (a.acc) {
      if (!launch) return occupancy<SRC, MODE, LVL, FIN_SSIM>();
      hipLaunchKernelGGL((ssim_mfma_kernel<SRC, MODE, LVL, FIN_SSIM>), grid, dim3(BLOCK), 0, st,
                         a);
      return 0;
    }
  }
  if (!launch) return occupancy<SRC, MODE, LVL>();
  hipLaunchKernelGGL((ssim_mfma_kernel<SRC, MODE, LVL>), grid, dim3(BLOCK), 0, st, a);
  return 0;
}

template <int SRC, int MODE>
int run_cs(bool launch, dim3 grid, hipStream_t st, const MfArgs& a) {
  if (!a.px) return run<SRC, MODE, LVL_NONE>(launch, grid, st, a);
  if constexpr (SRC == SRC_U8) {
    if (a.level_f16) return run<SRC, MODE, LVL_F16>(launch, grid, st, a);
  }
  return run<SRC, MODE, LVL_F32>(launch, grid, st, a);
}

// Pyramid levels come only through the CS pass (fa_gpu_ssim_cs_ex).
template <int SRC>
int dispatch(int mode, bool launch, dim3 grid, hipStream_t st, const MfArgs& a) {
  if (mode == MF_CS) return run_cs<SRC, MF_CS>(launch, grid, st, a);
  if (mode == MF_CSO) return run_cs<SRC, MF_CSO>(launch, grid, st, a);
  if constexpr (SRC == SRC_U8) {
    if (mode == MF_MAP) return run<SRC, MF_MAP, LVL_NONE>(launch, grid, st, a);
    return run<SRC, MF_REDUCE, LVL_NONE>(launch, grid, st, a);
  }
  return 0;
}

int dispatch(int src, int mode, bool launch, dim3 grid, hipStream_t st, const MfArgs& a) {
  return src == SRC_F32   ? dispatch<SRC_F32>(mode, launch, grid, st, a)
         : src == SRC_F16 ? dispatch<SRC_F16>(mode, launch, grid, st, a)
                          : dispatch<SRC_U8>(mode, launch, grid, st, a);
}

}  // namespace

namespace {

// The layout checks every matrix-core launch shares: rows and planes aligned
// to 8 samples, 4-byte (uint8) or 16-byte (levels) aligned bases, 16-byte
// aligned pyramid outputs, K <= 16, and the 32-bit offsets within a plane.
// uint8 samples are read as 8-byte buffer loads at multiples of 8 bytes from
// the base, so a 4-byte aligned base (a crop of 4 pixels, say) keeps every
// load dword-aligned, which is all a multi-dword buffer access requires.
bool mfma_fits(const SsimMfmaCall& c, int src, int mode) {
  if (c.K > MF_MAX_K || c.W % 8 != 0 || c.W < 8) return false;
  const uintptr_t base_align = src == SRC_U8 ? 3 : 15;
  if ((reinterpret_cast<uintptr_t>(c.x) | reinterpret_cast<uintptr_t>(c.y)) & base_align)
    return false;
  if (c.px && ((reinterpret_cast<uintptr_t>(c.px) | reinterpret_cast<uintptr_t>(c.py)) & 15))
    return false;
  const int64_t s[6] = {c.xsn, c.xsc, c.ysn, c.ysc, c.xsh, c.ysh};
  for (int64_t v : s)
    if (v % 8 != 0) return false;
  // the buffer loads run up to 47 rows past the last output row (their range
  // check stops them at the plane's end)
  const int64_t eb = src == SRC_F32 ? 4 : src == SRC_F16 ? 2 : 1;
  if ((static_cast<int64_t>(c.H) + 48) * std::max(c.xsh, c.ysh) * eb > INT32_MAX) return false;
  // the map is written through buffer resources with 32-bit offsets in a plane
  if (mode == MF_MAP && static_cast<int64_t>(c.Hout) * c.Wout * 4 > INT32_MAX) return false;
  return true;
}

MfArgs args_of(const SsimMfmaCall& c) {
  MfArgs a = {};
  a.x = c.x;
  a.y = c.y;
  a.xsn = c.xsn;
  a.xsc = c.xsc;
  a.ysn = c.ysn;
  a.ysc = c.ysc;
  a.xsh = static_cast<uint32_t>(c.xsh);
  a.ysh = static_cast<uint32_t>(c.ysh);
  a.C = c.C;
  a.H = c.H;
  a.W = c.W;
  a.Hout = c.Hout;
  a.Wout = c.Wout;
  a.K = c.K;
  a.win = c.win;
  a.C1 = static_cast<float>(c.C1);
  a.C2 = static_cast<float>(c.C2);
  a.one = 1.0f;
  a.map = c.map;
  a.partial = c.partial;
  a.partial_cs = c.partial_cs;
  a.px = c.px;
  a.py = c.py;
  a.level_f16 = c.level_f16 ? 1 : 0;
  return a;
}

// Rows per chunk (a multiple of 16): the fewest rounds of resident
// workgroups times the work of one, charging the extra 16-row block of
// horizontal work each chunk starts with at 10 rows, with at most max_tiles
// tiles per plane.  False when nothing fits.
//
// big_small: big chunks first, small ones last.  Workgroups start in tile
// order on each XCD, so the drain at the end of the launch -- the last
// workgroups running on emptying SIMDs -- lasts one small chunk instead of one
// of the uniform size.  Keeping the chunk count, the first half of a column's
// chunks get weight 1 and the rest 0.4 (on configs[1] 17,17,17,16 blocks
// become 24,24,10,9: 82.1 against 84.3 us per call over rotated input pairs,
// the same work and workgroup count).  It needs each XCD's range of tiles to
// hold whole planes (the count of planes a multiple of 8); walked plane by
// plane instead it measured slower.  A launch that fits one round of
// resident workgroups has no drain to shorten -- every chunk starts at once
// and the longest sets the time -- so it keeps uniform chunks.
bool plan_tiles(MfArgs& a, int64_t planes, int64_t resident, int64_t max_tiles,
                bool big_small) {
  const int strips = (a.Wout + WAVES_PER_BLOCK * MT - 1) / (WAVES_PER_BLOCK * MT);
  const int blocks = (a.Hout + MT - 1) / MT;
  int best_th = 0, best_chunks = 0;
  int64_t best_cost = INT64_MAX;
  for (int m = blocks; m >= 1; --m) {
    const int chunks = (blocks + m - 1) / m;
    if (static_cast<int64_t>(strips) * chunks > max_tiles) break;  // fewer rows: more tiles
    const int64_t wgs = planes * strips * chunks;
    const int64_t cost = ((wgs + resident - 1) / resident) * (MT * m + 10);
    if (cost < best_cost) {
      best_cost = cost;
      best_th = MT * m;
      best_chunks = chunks;
    }
  }
  if (best_th == 0) return false;
  a.TH = best_th;
  a.strips = strips;
  a.tiles = strips * best_chunks;
  a.nbig = best_chunks;
  a.THs = best_th;
  a.xcd_planes = 0;
  if (big_small && best_chunks >= 2 && planes % NUM_XCD == 0 &&
      planes * strips * best_chunks > resident) {
    const int nb = (best_chunks + 1) / 2;
    const int ns = best_chunks - nb;
    const int big = static_cast<int>(std::lround(blocks / (nb + 0.4 * ns)));
    if (big * nb < blocks) {
      const int small = (blocks - big * nb + ns - 1) / ns;
      const int chunks = nb + (blocks - big * nb + small - 1) / small;
      if (small >= 1 && small < big && static_cast<int64_t>(strips) * chunks <= max_tiles) {
        a.TH = MT * big;
        a.nbig = nb;
        a.THs = MT * small;
        a.tiles = strips * chunks;
        a.xcd_planes = static_cast<int>(planes / NUM_XCD);
      }
    }
  }
  return planes * a.tiles <= INT32_MAX;
}

// 2^F and 2^-F of a fixed-point sum of values in [-1, 1] over npix pixels:
// F = 51 - bits(2 npix) keeps the packed sum within its word.
void fixed_scale(double npix, double* fscale, double* finv) {
  int bits = 1;
  while (bits < 50 && std::ldexp(1.0, bits) <= 2.0 * npix) ++bits;
  *fscale = std::ldexp(1.0, 51 - bits);
  *finv = std::ldexp(1.0, bits - 51);
}

template <class K>
int occupancy_of(K kernel) {
  int v = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, reinterpret_cast<const void*>(kernel),
                                                   BLOCK, 0) != hipSuccess ||
      v <= 0)
    v = 1;
  return v;
}

}  // namespace

int ssim_mfma(const SsimMfmaCall& c, int device, hipStream_t st, int* tiles) {
  *tiles = 0;
  if (!mfma_enabled()) return FA_OK;
  const int src = c.src == SsimMfmaCall::F32_LEVEL   ? SRC_F32
                  : c.src == SsimMfmaCall::F16_LEVEL ? SRC_F16
                                                     : SRC_U8;
  // the CS pass, with (MF_CS) or without (MF_CSO, partial null) the SSIM sums
  const int mode = c.partial_cs ? (c.partial ? MF_CS : MF_CSO) : c.map ? MF_MAP : MF_REDUCE;
  const bool cs_pass = mode == MF_CS || mode == MF_CSO;
  if (src != SRC_U8 && !cs_pass) return FA_OK;
  if (c.level_f16 && (src != SRC_U8 || !cs_pass)) return FA_OK;
  if (!mfma_fits(c, src, mode)) return FA_OK;
  // the finish takes the uint8 forward's sums with a wanted output, where no
  // SSIM value can be NaN (C1, C2 > 0: with a zero constant a flat patch is
  // 0 / 0, which a fixed-point word cannot carry; the two-launch form's float64
  // sums pass it on, as the reference does)
  const bool fin = c.acc && src == SRC_U8 && mode == MF_REDUCE && c.N <= MF_FIN_MAX_IMAGES &&
                   (c.out_per_image || c.out_total) && c.C1 > 0.0 && c.C2 > 0.0;
  MfArgs a = args_of(c);
  const int occ = dispatch(src, mode, false, dim3(1), st, a);
  const int64_t planes = static_cast<int64_t>(c.N) * c.C;
  if (!plan_tiles(a, planes, static_cast<int64_t>(cu_count(device)) * occ, c.bpp, true))
    return FA_OK;
  const int64_t wgs = planes * a.tiles;
  // the one-launch finish, where its counts fit: C * tiles workgroups per
  // image and N images below 2^MF_COUNT_BITS (the tile plan above is the same
  // either way: the finish's kernel has the same occupancy)
  if (fin && static_cast<int64_t>(c.C) * a.tiles < (1 << MF_COUNT_BITS)) {
    a.acc = c.acc;
    a.out_per_image = c.out_per_image;
    a.out_total = c.out_total;
    a.N = c.N;
    a.npix_img = static_cast<double>(c.Hout) * c.Wout * c.C;
    a.npix_all = a.npix_img * c.N;
    int bits = 1;
    while (bits < 50 && std::ldexp(1.0, bits) <= 2.0 * a.npix_all) ++bits;
    a.fscale = std::ldexp(1.0, 51 - bits);
    a.finv = std::ldexp(1.0, bits - 51);
    if (bits >= 40) a.acc = nullptr;  // (never at real sizes) too few fraction bits left
  }
  // the forward's only launch without a workspace is the finish (the CS pass
  // forming the cs sums alone has a null `partial` of its own)
  if (!cs_pass && !a.acc && !c.partial) return FA_E_ARG;
  dispatch(src, mode, true, dim3(static_cast<unsigned>(wgs)), st, a);
  FA_LAUNCH_CHECK();
  *tiles = a.acc ? -1 : a.tiles;
  return FA_OK;
}

int ssim_mfma_ms(const SsimMfmaMs& c, int device, hipStream_t st, bool* done) {
  *done = false;
  const int M = c.M;
  const int64_t planes = static_cast<int64_t>(c.N) * c.C;
  if (!mfma_enabled() || !c.words || M < 3 || M > 2 + MS_TAIL_MAX) return FA_OK;
  if (planes > MS_FIN_MAX_PLANES || !(c.C1 > 0.0) || !(c.C2 > 0.0)) return FA_OK;
  if (!c.out_per_image && !c.out_total) return FA_OK;
  // every scale's call, checked before anything is launched
  MfArgs a[2 + MS_TAIL_MAX];
  double finv[MS_WORD_SCALES] = {}, npix[MS_WORD_SCALES] = {};
  int H = c.H, W = c.W;
  for (int i = 0; i < M; ++i) {
    SsimMfmaCall k = {};
    k.x = i == 0 ? c.x : c.lx[i];
    k.y = i == 0 ? c.y : c.ly[i];
    k.src = i == 0 ? SsimMfmaCall::U8 : i == 1 ? SsimMfmaCall::F16_LEVEL : SsimMfmaCall::F32_LEVEL;
    const int64_t plane = static_cast<int64_t>(H) * W;
    k.xsn = i == 0 ? c.xsn : plane * c.C;
    k.xsc = i == 0 ? c.xsc : plane;
    k.ysn = i == 0 ? c.ysn : plane * c.C;
    k.ysc = i == 0 ? c.ysc : plane;
    k.xsh = i == 0 ? c.xsh : W;
    k.ysh = i == 0 ? c.ysh : W;
    k.N = c.N;
    k.C = c.C;
    k.H = H;
    k.W = W;
    k.Hout = H - c.K + 1;
    k.Wout = W - c.K + 1;
    k.K = c.K;
    k.win = c.win;
    k.C1 = c.C1;
    k.C2 = c.C2;
    // the next level: float16 below the uint8 input, float32 below that
    if (i + 1 < M && i <= 1) {
      k.px = c.lx[i + 1];
      k.py = c.ly[i + 1];
      k.level_f16 = i == 0;
    }
    const int src = i == 0 ? SRC_U8 : i == 1 ? SRC_F16 : SRC_F32;
    if (k.Hout < 1 || k.Wout < 1 || !mfma_fits(k, src, i + 1 < M ? MF_CSO : MF_CS)) return FA_OK;
    if (i == 1)
      for (int d = 0; d < 2; ++d)
        if (3 + d < M && (reinterpret_cast<uintptr_t>(c.lx[3 + d]) |
                          reinterpret_cast<uintptr_t>(c.ly[3 + d])) & 15)
          return FA_OK;
    a[i] = args_of(k);
    npix[i] = static_cast<double>(k.Hout) * k.Wout;
    fixed_scale(npix[i], &a[i].fscale, &finv[i]);
    a[i].acc = c.words + static_cast<int64_t>(i) * planes * MF_STRIDE;
    H /= 2;
    W /= 2;
  }
  // scale 1 also writes the levels of scales 3 and 4
  for (int d = 0; d < 2; ++d) {
    a[1].dpx[d] = 3 + d < M ? c.lx[3 + d] : nullptr;
    a[1].dpy[d] = 3 + d < M ? c.ly[3 + d] : nullptr;
  }
  const int64_t cus = cu_count(device);
  auto k0 = ssim_mfma_kernel<SRC_U8, MF_CSO, LVL_F16, FIN_MS>;
  auto k1 = ssim_mfma_kernel<SRC_F16, MF_CSO, LVL_F32D, FIN_MS>;
  static const int occ0 = occupancy_of(k0), occ1 = occupancy_of(k1),
                   occt = occupancy_of(ssim_mfma_tail_kernel);
  // the counts of every word (tiles per plane) stay below 2^MF_COUNT_BITS
  constexpr int64_t max_tiles = (1 << MF_COUNT_BITS) - 1;
  if (!plan_tiles(a[0], planes, cus * occ0, max_tiles, true) ||
      !plan_tiles(a[1], planes, cus * occ1, max_tiles, true))
    return FA_OK;
  // The coarse scales share one round of resident workgroups: starting from
  // one chunk per column, the scale with the longest chunks is split once
  // more while the launch still fits the round (on configs[4]: 3, 1 and 2
  // chunks, 720 of 768 workgroups).  Measured: these passes are bound by
  // instruction issue, so more workgroups than the round holds only add the
  // extra block of rows each chunk starts with; planned one scale at a time
  // (each with the whole round) the launch took 27.6 us, planned together
  // 22-24.
  MfTail t = {};
  t.n = M - 2;
  t.first = 2;
  int chunks[MS_TAIL_MAX], blocks[MS_TAIL_MAX];
  int64_t cols[MS_TAIL_MAX], wgs = 0;
  for (int k = 0; k < t.n; ++k) {
    MfArgs& s = a[2 + k];
    s.strips = (s.Wout + WAVES_PER_BLOCK * MT - 1) / (WAVES_PER_BLOCK * MT);
    blocks[k] = (s.Hout + MT - 1) / MT;
    cols[k] = planes * s.strips;
    chunks[k] = 1;
    wgs += cols[k];
  }
  const int64_t round = cus * occt;
  for (;;) {
    int pick = -1, longest = 0;
    for (int k = 0; k < t.n; ++k) {
      const int len = (blocks[k] + chunks[k] - 1) / chunks[k];
      if (len > 1 && len > longest && wgs + cols[k] <= round) {
        longest = len;
        pick = k;
      }
    }
    if (pick < 0) break;
    ++chunks[pick];
    wgs += cols[pick];
  }
  wgs = 0;
  for (int k = 0; k < t.n; ++k) {
    MfArgs& s = a[2 + k];
    const int m = (blocks[k] + chunks[k] - 1) / chunks[k];  // blocks per chunk
    const int ch = (blocks[k] + m - 1) / m;
    s.TH = s.THs = MT * m;
    s.nbig = ch;
    s.tiles = s.strips * ch;
    s.xcd_planes = 0;
    if (s.tiles > max_tiles) return FA_OK;
    wgs += planes * s.tiles;
    if (wgs > INT32_MAX) return FA_OK;
    t.s[k] = s;
    t.wg_end[k] = static_cast<int>(wgs);
  }
  t.M = M;
  t.N = c.N;
  t.C = c.C;
  t.planes = static_cast<int>(planes);
  t.words = c.words;
  for (int i = 0; i < M; ++i) {
    t.finv[i] = finv[i];
    t.npix[i] = npix[i];
    t.w[i] = c.weights[i];
  }
  t.out_per_image = c.out_per_image;
  t.out_total = c.out_total;
  hipLaunchKernelGGL(k0, dim3(static_cast<unsigned>(planes * a[0].tiles)), dim3(BLOCK), 0, st,
                     a[0]);
  FA_LAUNCH_CHECK();
  hipLaunchKernelGGL(k1, dim3(static_cast<unsigned>(planes * a[1].tiles)), dim3(BLOCK), 0, st,
                     a[1]);
  FA_LAUNCH_CHECK();
  hipLaunchKernelGGL(ssim_mfma_tail_kernel, dim3(static_cast<unsigned>(wgs)), dim3(BLOCK), 0,
                     st, t);
  FA_LAUNCH_CHECK();
  *done = true;
  return FA_OK;
}

}  // namespace fa
