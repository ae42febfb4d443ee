// GMSD / GMS on gfx950: optional 2x2 mean downsample, 3x3 Prewitt pair (taps
// +-1/3, 'valid' support), gradient-magnitude similarity
//     g = sqrt(gx^2 + gy^2 + eps),  q = (2 g1 g2 + T) / (g1^2 + g2^2 + T)
// and the per-image mean and population standard deviation of q
// (reference: fa_cuda.cu:926-1026, 1416-1466; reference.py:288-335).
//
// Layout on CDNA4.  A wave walks a strip of 64 * NC sample columns (NC per
// lane) top to bottom with a three-row window in registers and the next rows'
// loads in flight; the Prewitt neighbours to the right come from in-wave
// shuffles.  No LDS and no barriers, so every wave is independent.  The four
// waves of a workgroup take four adjacent strips over the same rows (one
// contiguous stretch of each input row), and the launch is exactly one round
// of resident workgroups: each takes an equal share of its image's (channel,
// strip group, row) space, a run of rows that may continue into the next
// group or channel with a fresh two-row window.  Every workgroup does the
// same work (to a row), so there is no tail, and the re-read halo is two rows
// per run.  Loads beyond a run are clamped to its last row rather than
// branched around, which keeps the double-buffered loads in flight.
//
// Arithmetic.  Samples are kept unnormalised: the sum of a 2x2 block (or the
// sample itself), so for uint8 input they are integers and the Prewitt sums,
// differences and M = (3 s gx)^2 + (3 s gy)^2 are exact int32 (s = 4 with
// downsampling, else 1).  With G = M + 9 s^2 eps and T' = 9 s^2 T the kernel
// accumulates not q but
//     d = 1 - q = (g1 - g2)^2 / (G1 + G2 + T')
//              = (M1 - M2)^2 / ((G1 + G2 + 2 sqrt(G1 G2)) (G1 + G2 + T'))
// whose numerator is an exact integer for uint8.  Every rounding after it is
// then *relative* to d, so it scales the variance instead of being amplified
// by the difference E[q^2] - E[q]^2 of two numbers near 1 (an absolute error
// of e in q moves the deviation by ~e / var(q), i.e. ~1e4 e).  Where the
// sample magnitudes are bounded (uint8, float16) d is formed in float32 with
// v_sqrt_f32 / v_rcp_f32 (a few ulp, relative); other inputs form it in
// float64.  Sum d and sum d^2 are float64, reduced in a fixed order; the
// finalize returns mean q = 1 - mean d and std q = std d.
//
// Luma (an extension): with per-channel weights the kernel reads the three
// channels of each pixel and forms kr R + kg G + kb B itself, in float64,
// instead of a float32 luma plane materialised beforehand.  A luma offset
// cancels out of every gradient, so it is not an argument.
#include "fa_common.h"

#include <algorithm>
#include <type_traits>

namespace fa {

constexpr int G_PD = 2;        // rows of loads in flight ahead of the window
constexpr int G_MIN_ROWS = 8;  // fewest rows a wave is given, where rows are scarce
constexpr int G_SLOT_ROWS = 4; // workspace: one partial slot per 4 rows of a strip
constexpr int G_OUTW_WIDE = 2 * WAVE - 2;  // output columns per wave, 2 columns per lane
constexpr int G_OUTW_NARROW = WAVE - 2;    // ... 1 column per lane
// at most this many waves per SIMD in the one round of resident waves: more
// waves give each wave a shorter run, whose prologue (two window rows, the
// first loads' latency) and final reductions then weigh more; measured
// slower at 7 and 8 on configs[4]
constexpr int G_MAX_WAVES_PER_SIMD = 6;

struct GView {
  int64_t sn, sc, sh;  // element strides of image, channel, row (columns are unit stride)
};

struct GmsdArgs {
  const void* x;
  const void* y;
  GView vx, vy;
  int Cout;                  // output planes per image (1 with luma)
  int Hd, Wd, Hout, Wout;    // sample grid and 'valid' output grid
  int strips;                // strips per plane
  int groups;                // strip groups per plane: the 4 waves of a workgroup
  int wpi;                   // workgroups per image
  int tasks;                 // N * wpi
  int64_t rows_img;          // Cout * groups * Hout: an image's row space
  double kr, kg, kb;         // luma weights
  double T2, eps2;           // T and eps scaled by 9 s^2
  float T2f, eps2f;
  int ext_x, ext_y;          // bytes from a plane's base to its last byte + 1 (dword path)
  double* psum;
  double* psumsq;
  float* map;                // optional q map, [N * Cout, Hout, Wout]
  // the one-launch finish (gmsd_kernel<..., FIN>): accumulator words, the
  // fixed-point scale 2^F of the per-image sums and its inverse, and outputs
  uint64_t* acc;
  double fscale, finv, npix;
  double *out_mean, *out_std, *out_batch;
  int N;
};

// d = 1 - q from the squared gradient magnitudes M1, M2 (without eps) and
// their difference dm = M1 - M2 (exact for integer samples).  float32 where
// FAST, else float64.
template <bool FAST, typename S>
__device__ inline typename std::conditional<FAST, float, double>::type one_minus_q(
    S m1, S m2, S dm, float e_f, float t_f, double e_d, double t_d) {
  if constexpr (FAST) {
    const float f1 = static_cast<float>(m1), f2 = static_cast<float>(m2);
    const float G1 = f1 + e_f;
    const float G2 = f2 + e_f;
    const float Gs = G1 + G2;
    const float A = fmaf(2.0f, __builtin_amdgcn_sqrtf(G1 * G2), Gs);  // (g1 + g2)^2
    // integer magnitudes below 2^24 are exact in float32, so f1 - f2 is dm;
    // above, both gradients are near their maximum, the rounding moves dm by
    // at most 2, and where that is a large share of dm, d is below 1e-14.
    // Other sources pass dm exactly.
    const float n = std::is_integral<S>::value ? f1 - f2 : static_cast<float>(dm);
    // positive e_f and t_f arrive floored at 1e-18 (gmsd_impl), so where
    // either is positive A (Gs + t_f) >= 1e-36, a normal float32, and the
    // reciprocal is finite; with both zero a flat pixel's 0 * rcp(0) is NaN,
    // the reference's 0 / 0
    return (n * n) * __builtin_amdgcn_rcpf(A * (Gs + t_f));
  } else {
    const double G1 = static_cast<double>(m1) + e_d;
    const double G2 = static_cast<double>(m2) + e_d;
    const double Gs = G1 + G2;
    const double A = fma(2.0, sqrt(G1 * G2), Gs);
    const double n = static_cast<double>(dm);
    return (n * n) / (A * (Gs + t_d));  // 0 / 0 = NaN on a flat patch with T = eps = 0
  }
}

// Buffer-resource word 3 for raw (untyped, unswizzled) dword access on CDNA.
constexpr int G_RSRC_WORD3 = 0x00020000;

// --------------------------------------------------------------------------
// sample sources: what one lane loads for one sample row, and the samples
// --------------------------------------------------------------------------

// uint8, 2x2 downsampling, 4-byte aligned rows: each lane owns two sample
// columns (four input bytes per input row) and loads them as one dword.
// Channel sums are integers formed by v_dot4_u32_u8.
template <bool LUMA>
struct SrcU8Wide {
  static constexpr int NC = 2;
  static constexpr int OUTW = G_OUTW_WIDE;
  static constexpr int CH = LUMA ? 3 : 1;
  static constexpr bool FAST = true;
  static constexpr bool PACKED = !LUMA;  // samples_xy / prewitt_xy
  using S = typename std::conditional<LUMA, double, int>::type;
  struct Raw {
    uint32_t w[2][CH][2];  // tensor, channel, input row of the pair
  };

  // Buffer resources on the channel planes of x / y for this image (range:
  // the plane's extent): a row is a scalar offset and the lane a 32-bit
  // vector offset, so a load costs no VALU address arithmetic.  Rows and
  // column pairs are clamped, so every access is inside the plane.
  __amdgpu_buffer_rsrc_t rx[CH], ry[CH];
  uint32_t shx, shy;
  int rlo, rlim;  // first and last sample row a load may touch (clamp)
  uint32_t boff;  // this lane's byte offset in a row
  double kr, kg, kb;

  __device__ inline void setup(const GmsdArgs& a, int n, int c, int strip, int lane) {
    const uint8_t* bx = static_cast<const uint8_t*>(a.x) + n * a.vx.sn;
    const uint8_t* by = static_cast<const uint8_t*>(a.y) + n * a.vy.sn;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
      rx[ch] = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(bx + (LUMA ? ch : c) * a.vx.sc), 0, a.ext_x, G_RSRC_WORD3);
      ry[ch] = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(by + (LUMA ? ch : c) * a.vy.sc), 0, a.ext_y, G_RSRC_WORD3);
    }
    shx = static_cast<uint32_t>(a.vx.sh);
    shy = static_cast<uint32_t>(a.vy.sh);
    rlo = 0;
    rlim = a.Hd - 1;
    int pair = strip * (OUTW / 2) + lane;  // covers sample columns 2 pair, 2 pair + 1
    const int last = a.Wd / 2 - 1;         // Wd is even on this path
    boff = 4u * static_cast<uint32_t>(pair < last ? pair : last);
    kr = a.kr;
    kg = a.kg;
    kb = a.kb;
  }

  __device__ inline Raw load(int r) const {
    const int rc = r < rlo ? rlo : (r < rlim ? r : rlim);
    const uint32_t ir = 2u * static_cast<uint32_t>(rc);
    const int ox = static_cast<int>(ir * shx), oy = static_cast<int>(ir * shy);
    Raw v;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
      v.w[0][ch][0] = __builtin_amdgcn_raw_buffer_load_b32(rx[ch], boff, ox, 0);
      v.w[0][ch][1] = __builtin_amdgcn_raw_buffer_load_b32(rx[ch], boff, ox + static_cast<int>(shx), 0);
      v.w[1][ch][0] = __builtin_amdgcn_raw_buffer_load_b32(ry[ch], boff, oy, 0);
      v.w[1][ch][1] = __builtin_amdgcn_raw_buffer_load_b32(ry[ch], boff, oy + static_cast<int>(shy), 0);
    }
    return v;
  }

  __device__ inline void samples(const Raw& v, S (&sx)[NC], S (&sy)[NC]) const {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      int s[CH][NC];
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        s[ch][0] = static_cast<int>(__builtin_amdgcn_udot4(
            v.w[t][ch][1], 0x00000101u, __builtin_amdgcn_udot4(v.w[t][ch][0], 0x00000101u, 0u, false), false));
        s[ch][1] = static_cast<int>(__builtin_amdgcn_udot4(
            v.w[t][ch][1], 0x01010000u, __builtin_amdgcn_udot4(v.w[t][ch][0], 0x01010000u, 0u, false), false));
      }
      S* o = t ? sy : sx;
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        if constexpr (LUMA)
          o[k] = fma(kb, static_cast<double>(s[2][k]),
                     fma(kg, static_cast<double>(s[1][k]), kr * static_cast<double>(s[0][k])));
        else
          o[k] = s[0][k];
      }
    }
  }

  // Column k's x sample in the low 16 bits of p[k], its y sample in the high
  // 16 (each at most 4 * 255, so neither half carries into the other).  The x
  // sample is two byte dot products; the y sample gathers its four bytes (two
  // of each input row) with one byte permute and adds their sum, shifted up
  // 16, to the x sample in one v_sad_hi_u8 (sum of |byte - 0| << 16, plus
  // the accumulator).
  __device__ inline void samples_xy(const Raw& v, uint32_t (&p)[NC]) const {
    static_assert(!LUMA && NC == 2, "packed samples: uint8, two columns per lane");
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const uint32_t wk = k ? 0x01010000u : 0x00000101u;
      const uint32_t sx = __builtin_amdgcn_udot4(v.w[0][0][1], wk,
                                                 __builtin_amdgcn_udot4(v.w[0][0][0], wk, 0u, false), false);
      const uint32_t yb = __builtin_amdgcn_perm(v.w[1][0][1], v.w[1][0][0], k ? 0x07060302u : 0x05040100u);
      p[k] = __builtin_amdgcn_sad_hi_u8(yb, 0u, sx);
    }
  }
};

// Any element type, with or without downsampling, any strides: one sample
// column per lane, float64 samples (exact sums for every 8/16/32-bit input).
template <typename T, bool DOWN, bool LUMA>
struct SrcGeneric {
  static constexpr int NC = 1;
  static constexpr int OUTW = G_OUTW_NARROW;
  static constexpr int CH = LUMA ? 3 : 1;
  static constexpr int NV = DOWN ? 4 : 1;
  static constexpr bool FAST = std::is_same<T, uint8_t>::value || std::is_same<T, half_t>::value;
  static constexpr bool PACKED = false;
  using S = double;
  struct Raw {
    T v[2][CH][NV];
  };

  const T* px[CH];
  const T* py[CH];
  int64_t shx, shy;
  int rlo, rlim;  // first and last sample row a load may touch (clamp)
  uint32_t col;  // first input column of this lane's sample
  double kr, kg, kb;

  __device__ inline void setup(const GmsdArgs& a, int n, int c, int strip, int lane) {
    const T* bx = static_cast<const T*>(a.x) + n * a.vx.sn;
    const T* by = static_cast<const T*>(a.y) + n * a.vy.sn;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
      px[ch] = bx + (LUMA ? ch : c) * a.vx.sc;
      py[ch] = by + (LUMA ? ch : c) * a.vy.sc;
    }
    shx = a.vx.sh;
    shy = a.vy.sh;
    rlo = 0;
    rlim = a.Hd - 1;
    const int sc = strip * OUTW + lane;
    col = static_cast<uint32_t>(DOWN ? 2 * (sc < a.Wd ? sc : a.Wd - 1) : (sc < a.Wd ? sc : a.Wd - 1));
    kr = a.kr;
    kg = a.kg;
    kb = a.kb;
  }

  __device__ inline Raw load(int r) const {
    const int rr = r < rlo ? rlo : (r < rlim ? r : rlim);
    const int64_t ir = DOWN ? 2 * static_cast<int64_t>(rr) : rr;
    Raw v;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
      const T* rx = px[ch] + ir * shx + col;
      const T* ry = py[ch] + ir * shy + col;
      v.v[0][ch][0] = rx[0];
      v.v[1][ch][0] = ry[0];
      if constexpr (DOWN) {
        v.v[0][ch][1] = rx[1];
        v.v[0][ch][2] = rx[shx];
        v.v[0][ch][3] = rx[shx + 1];
        v.v[1][ch][1] = ry[1];
        v.v[1][ch][2] = ry[shy];
        v.v[1][ch][3] = ry[shy + 1];
      }
    }
    return v;
  }

  __device__ inline void samples(const Raw& v, S (&sx)[NC], S (&sy)[NC]) const {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      double s[CH];
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) {
        s[ch] = Elem<T>::d(v.v[t][ch][0]);
        if constexpr (DOWN)
          s[ch] = (s[ch] + Elem<T>::d(v.v[t][ch][1])) +
                  (Elem<T>::d(v.v[t][ch][2]) + Elem<T>::d(v.v[t][ch][3]));
      }
      S* o = t ? sy : sx;
      if constexpr (LUMA)
        o[0] = fma(kb, s[2], fma(kg, s[1], kr * s[0]));
      else
        o[0] = s[0];
    }
  }
};

// --------------------------------------------------------------------------
// one wave: one (plane, chunk, strip) task
// --------------------------------------------------------------------------

// 3 s gx and 3 s gy at this lane's NC columns from the window rows a (top),
// b, c (bottom).
template <typename S, int NC>
__device__ inline void prewitt(const S (&a)[NC], const S (&b)[NC], const S (&c)[NC],
                               S (&gx)[NC], S (&gy)[NC]) {
  S cs[NC + 2], rd[NC + 2];  // this lane's columns, then the next lane's first two
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    cs[k] = a[k] + b[k] + c[k];  // column sums, differenced across for gx
    rd[k] = a[k] - c[k];         // row differences, summed across for gy
  }
  // neighbours by DPP; the last lanes' are zero, and those lanes' columns lie
  // past the strip's output (masked by the caller)
  if constexpr (NC >= 2) {
    cs[NC] = wave_next(cs[0]);
    cs[NC + 1] = wave_next(cs[1]);
    rd[NC] = wave_next(rd[0]);
    rd[NC + 1] = wave_next(rd[1]);
  } else {
    cs[2] = wave_next(wave_next(cs[0]));
    rd[1] = wave_next(rd[0]);
    rd[2] = wave_next(rd[1]);
  }
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    gx[k] = cs[k] - cs[k + 2];
    gy[k] = rd[k] + rd[k + 1] + rd[k + 2];
  }
}

// M1, M2 and M1 - M2.  Integer components are below 2^13 in magnitude, so the
// 24-bit multiplier (full rate) is exact; float64 components use the
// factored difference, which keeps dm accurate when M1 ~ M2.
__device__ inline void mag2(int gx1, int gy1, int gx2, int gy2, int& m1, int& m2, int& dm) {
  m1 = __mul24(gx1, gx1) + __mul24(gy1, gy1);
  m2 = __mul24(gx2, gx2) + __mul24(gy2, gy2);
  dm = m1 - m2;
}
// The Prewitt responses of both tensors at once: column k's samples of x and y
// share one register (x low, y high half; see samples_xy), and the column
// sums, row differences and their neighbours are formed on both halves by
// packed 16-bit operations.  Every intermediate fits in int16: samples are at
// most 1020, column sums 3060, row differences, gx and gy within +-3060.
// M1 (x) and M2 (y) are then dot products of [gx, gy] with itself (the two
// halves regathered by a byte permute), exact in int32.
using short2_t = short __attribute__((ext_vector_type(2)));
// v . v of two int16 lanes; the three-operand form with an inline zero (the
// builtin's accumulating two-operand form costs a zeroing move per use)
__device__ inline int sdot2_self(uint32_t v) {
  int r;
  asm("v_dot2_i32_i16 %0, %1, %1, 0" : "=v"(r) : "v"(v));
  return r;
}
// a + b + c in one instruction (the compiler prefers two adds sharing a pair
// sum across rows; on gfx950 every vector instruction of mixed code costs
// about the same, so one is cheaper)
__device__ inline uint32_t add3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_add3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ inline void prewitt_xy(const uint32_t (&a)[2], const uint32_t (&b)[2],
                                  const uint32_t (&c)[2], int (&m1)[2], int (&m2)[2]) {
  uint32_t cs[2];
  short2_t rd[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    cs[k] = add3_u32(a[k], b[k], c[k]);
    rd[k] = __builtin_bit_cast(short2_t, a[k]) - __builtin_bit_cast(short2_t, c[k]);
  }
  // the next lane's two columns (zero past the wave: those columns are masked)
  const short2_t ncs0 = __builtin_bit_cast(short2_t, wave_next(static_cast<int>(cs[0])));
  const short2_t ncs1 = __builtin_bit_cast(short2_t, wave_next(static_cast<int>(cs[1])));
  const short2_t nrd0 = __builtin_bit_cast(short2_t, wave_next(__builtin_bit_cast(int, rd[0])));
  const short2_t nrd1 = __builtin_bit_cast(short2_t, wave_next(__builtin_bit_cast(int, rd[1])));
  const short2_t gx0 = __builtin_bit_cast(short2_t, cs[0]) - ncs0;
  const short2_t gx1 = __builtin_bit_cast(short2_t, cs[1]) - ncs1;
  const short2_t t = rd[1] + nrd0;
  const short2_t gy0 = rd[0] + t, gy1 = t + nrd1;
  const short2_t gx[2] = {gx0, gx1}, gy[2] = {gy0, gy1};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, gx[k]), uy = __builtin_bit_cast(uint32_t, gy[k]);
    const short2_t vx = __builtin_bit_cast(short2_t, __builtin_amdgcn_perm(uy, ux, 0x05040100u));
    const short2_t vy = __builtin_bit_cast(short2_t, __builtin_amdgcn_perm(uy, ux, 0x07060302u));
    m1[k] = sdot2_self(__builtin_bit_cast(uint32_t, vx));
    m2[k] = sdot2_self(__builtin_bit_cast(uint32_t, vy));
  }
}

__device__ inline void mag2(double gx1, double gy1, double gx2, double gy2, double& m1,
                            double& m2, double& dm) {
  m1 = fma(gx1, gx1, gy1 * gy1);
  m2 = fma(gx2, gx2, gy2 * gy2);
  dm = fma(gx1 - gx2, gx1 + gx2, (gy1 - gy2) * (gy1 + gy2));
}

// Rows [row0, row0 + rows) of one strip of one plane, added to acc / acc2,
// walked top-down, or bottom-up when `up` (uniform).  Walking up swaps the
// window's top and bottom rows, which only flips the sign of gy: the
// magnitudes, and so every term, are the same.  MAP: also write the q map.
template <class Src, bool MAP>
__device__ inline void gmsd_run(const GmsdArgs& a, int n, int c, int strip, int row0, int rows,
                                bool up, double& acc, double& acc2) {
  float* const map_plane =
      MAP ? a.map + (static_cast<int64_t>(n) * a.Cout + c) * a.Hout * a.Wout : nullptr;
  using S = typename Src::S;
  using Raw = typename Src::Raw;
  constexpr int NC = Src::NC;
  const int lane = threadIdx.x % WAVE;

  Src src;
  src.setup(a, n, c, strip, lane);
  // Loads past the run re-read its last row (cached) instead of being
  // branched around: a conditional load group makes the compiler wait for
  // every load in flight, which would serialise the double buffering.
  src.rlo = row0;
  src.rlim = row0 + rows + 1;
  // sample row of step j of the walk (the window's newest row)
  auto srow = [&](int j) { return up ? row0 + rows + 1 - j : row0 + j; };
  const int col = strip * Src::OUTW + NC * lane;  // first output column of the lane
  bool ok[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) ok[k] = NC * lane + k < Src::OUTW && col + k < a.Wout;

  // every load of the prologue is in flight before the first one is used
  const Raw p0 = src.load(srow(0)), p1 = src.load(srow(1));
  // two named row buffers, so a group never copies the one in flight
  Raw bufA[G_PD], bufB[G_PD];
#pragma unroll
  for (int i = 0; i < G_PD; ++i) bufA[i] = src.load(srow(2 + i));
  S xa[NC], xb[NC], ya[NC], yb[NC];
  uint32_t pa[NC], pb[NC];  // PACKED: x and y samples of a column in one register
  if constexpr (Src::PACKED) {
    src.samples_xy(p0, pa);
    src.samples_xy(p1, pb);
  } else {
    src.samples(p0, xa, ya);
    src.samples(p1, xb, yb);
  }

  using Acc = typename std::conditional<Src::FAST, float, double>::type;
  // G_PD rows from `cur`, starting at row g of the run (FULL: all G_PD lie in
  // the run, so the body has no row test and the window rotates by renaming).
  // Each column sums its own terms; a lane's columns past the strip or the
  // image (ok false) hold finite garbage that the group drops once, by
  // selection, instead of masking every term.  The sums are formed at the
  // accumulation type, then added in float64.
  auto group = [&](const Raw (&cur)[G_PD], int g, auto full) {
    Acc gs[NC], gs2[NC];  // -0 + d is d exactly, so the first add folds away
#pragma unroll
    for (int k = 0; k < NC; ++k) gs[k] = gs2[k] = Acc(-0.0);
#pragma unroll
    for (int i = 0; i < G_PD; ++i) {
      if (decltype(full)::value || g + i < rows) {  // uniform
        S m1[NC], m2[NC], dm[NC];
        if constexpr (Src::PACKED) {
          uint32_t pc[NC];
          src.samples_xy(cur[i], pc);
          prewitt_xy(pa, pb, pc, m1, m2);
#pragma unroll
          for (int k = 0; k < NC; ++k) {
            dm[k] = m1[k] - m2[k];
            pa[k] = pb[k];
            pb[k] = pc[k];
          }
        } else {
          S xc[NC], yc[NC];
          src.samples(cur[i], xc, yc);
          S gx1[NC], gy1[NC], gx2[NC], gy2[NC];
          prewitt<S, NC>(xa, xb, xc, gx1, gy1);
          prewitt<S, NC>(ya, yb, yc, gx2, gy2);
#pragma unroll
          for (int k = 0; k < NC; ++k) {
            mag2(gx1[k], gy1[k], gx2[k], gy2[k], m1[k], m2[k], dm[k]);
            xa[k] = xb[k];
            xb[k] = xc[k];
            ya[k] = yb[k];
            yb[k] = yc[k];
          }
        }
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          const Acc d = one_minus_q<Src::FAST, S>(m1[k], m2[k], dm[k], a.eps2f, a.T2f, a.eps2, a.T2);
          if constexpr (MAP) {
            if (ok[k])
              map_plane[static_cast<int64_t>(up ? row0 + rows - 1 - g - i : row0 + g + i) *
                            a.Wout + col + k] = static_cast<float>(1.0 - static_cast<double>(d));
          }
          gs[k] += d;
          gs2[k] = fma(d, d, gs2[k]);
        }
      }
    }
    Acc s = Acc(0), s2 = Acc(0);
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      s += ok[k] ? gs[k] : Acc(0);
      s2 += ok[k] ? gs2[k] : Acc(0);
    }
    acc += static_cast<double>(s);
    acc2 += static_cast<double>(s2);
  };

  for (int g = 0; g < rows; g += 2 * G_PD) {
#pragma unroll
    for (int i = 0; i < G_PD; ++i) bufB[i] = src.load(srow(2 + g + G_PD + i));
    if (g + G_PD <= rows)
      group(bufA, g, std::true_type{});
    else
      group(bufA, g, std::false_type{});
    if (g + G_PD >= rows) break;
#pragma unroll
    for (int i = 0; i < G_PD; ++i) bufA[i] = src.load(srow(2 + g + 2 * G_PD + i));
    if (g + 2 * G_PD <= rows)
      group(bufB, g + G_PD, std::true_type{});
    else
      group(bufB, g + G_PD, std::false_type{});
  }
}

// --------------------------------------------------------------------------
// The one-launch finish (fa_gpu_gmsd_once), with T or eps positive, where the
// d = 1 - q of finite samples are in [0, 1].
//
// A workgroup's sums of d and d^2 go to two accumulator words of its image as
// fixed-point integers, round(sum * 2^F) with F = 52 - bits(pixels per image
// + 1), packed with a contribution count: word = (value << GF_COUNT_BITS) +
// count.  One returning device-scope atomic per word adds both at once, and
// integer addition does not depend on the order, so the result is the same
// from run to run.  The workgroup whose add brings a word's count to the
// image's workgroup count holds that word's complete sum.  The two words of
// an image may be completed by different workgroups, which meet on a third
// word: each exchanges its completed value (with a presence bit and a bit
// saying which sum it is) into it, and the one that gets the other's value
// back holds both, writes the image's mean q = 1 - mean d and population
// std q = std d, and resets the meeting word.  It then adds the two results,
// in fixed point with 2^45, to two batch words counted in images, whose
// finishers write the batch means.  Every word is reset to zero by the one
// that completes it, so the buffer is zero again when the call ends.  Words
// sit on their own 128-byte lines.
//
// Each workgroup's rounding is at most 2^-(F+1) on a sum below 2^(52-F), so
// the per-image sums keep ~2^-52 relative accuracy times the workgroup count.
//
// Floating input can hold NaN or inf, which make d NaN; a fixed-point word
// cannot carry it.  A lane whose sum is not finite adds 0 and first sets a
// flag, the second word of the image's meeting line, with a returning atomic
// it waits for; the meeting's completer, whose view has every add of both
// words behind it (and so every flag set before them), reads and clears the
// flag by an exchange and writes NaN for both statistics, as the reference's
// float statistics would be; the batch words carry flags the same way.
// --------------------------------------------------------------------------
constexpr int GF_COUNT_BITS = 12;  // workgroups per image: < 4096
constexpr int GF_STRIDE = 16;      // uint64 words between accumulators (128 bytes)
constexpr int GF_MAX_IMAGES = 64;
constexpr int GF_BATCH_BITS = 45;  // fixed-point bits of the batch sums (<= 64 images in [0, 1])
constexpr uint64_t GF_PRESENT = uint64_t(1) << 62;
constexpr uint64_t GF_IS_SQ = uint64_t(1) << 61;
static_assert(FA_GMSD_ACC_WORDS == (3 * GF_MAX_IMAGES + 2) * GF_STRIDE,
              "the ABI's accumulator size");

__device__ inline uint64_t gf_add(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t gf_swap(uint64_t* p, uint64_t v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void gf_zero(uint64_t* p) {
  __hip_atomic_store(p, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// Mean q and population std q of an image from its sums of d = 1 - q.  A NaN
// variance (a NaN q, e.g. a flat patch with T = eps = 0) stays NaN.
__device__ inline void gmsd_stats(double sa, double sb, double npix, double* mean,
                                  double* sd) {
  const double md = sa / npix;  // mean of d = 1 - q
  const double var = sb / npix - md * md;
  *mean = 1.0 - md;
  *sd = sqrt(var < 0.0 ? 0.0 : var);
}

// Lane `which` (0: sum d, 1: sum d^2) of image n adds the workgroup's `v`.
__device__ inline void gmsd_finish(const GmsdArgs& a, int n, int which, double v) {
  constexpr uint64_t CM = (uint64_t(1) << GF_COUNT_BITS) - 1;
  constexpr double NaN = __builtin_nan("");
  uint64_t* w = a.acc + static_cast<int64_t>(3 * n + which) * GF_STRIDE;
  uint64_t* meet = a.acc + static_cast<int64_t>(3 * n + 2) * GF_STRIDE;
  const bool finite = __builtin_isfinite(v);
  if (!finite) fin_flag_set(meet + 1);
  const uint64_t f = finite ? static_cast<uint64_t>(__double2ll_rn(v * a.fscale)) : 0u;
  const uint64_t old = gf_add(w, (f << GF_COUNT_BITS) + 1u);
  if ((old & CM) + 1u != static_cast<uint64_t>(a.wpi)) return;
  gf_zero(w);
  const uint64_t mine = (old >> GF_COUNT_BITS) + f;
  const uint64_t other = gf_swap(meet, mine | GF_PRESENT | (which ? GF_IS_SQ : 0));
  if (!(other & GF_PRESENT)) return;  // the other sum is not complete yet
  gf_zero(meet);
  const bool nan_img = fin_flag_take(meet + 1);
  const uint64_t ov = other & (GF_IS_SQ - 1);
  const double sd = static_cast<double>(which ? ov : mine) * a.finv;
  const double sd2 = static_cast<double>(which ? mine : ov) * a.finv;
  double mq, sq;
  gmsd_stats(sd, sd2, a.npix, &mq, &sq);
  if (nan_img) mq = sq = NaN;
  a.out_mean[n] = mq;
  a.out_std[n] = sq;
  if (!a.out_batch) return;
  const double bs = static_cast<double>(uint64_t(1) << GF_BATCH_BITS);
  const double r[2] = {mq, sq};
  uint64_t* b[2];
  uint64_t fb[2], ob[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    b[k] = a.acc + static_cast<int64_t>(3 * GF_MAX_IMAGES + k) * GF_STRIDE;
    if (nan_img) fin_flag_set(b[k] + 1);
    fb[k] = nan_img ? 0u : static_cast<uint64_t>(__double2ll_rn(r[k] * bs));
  }
  // both batch adds in flight at once: neither waits for the other's return
#pragma unroll
  for (int k = 0; k < 2; ++k) ob[k] = gf_add(b[k], (fb[k] << GF_COUNT_BITS) + 1u);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if ((ob[k] & CM) + 1u != static_cast<uint64_t>(a.N)) continue;
    gf_zero(b[k]);
    const bool nan_all = fin_flag_take(b[k] + 1);
    a.out_batch[k] =
        nan_all ? NaN : static_cast<double>((ob[k] >> GF_COUNT_BITS) + fb[k]) / bs / a.N;
  }
}

template <class Src, bool MAP, bool FIN = false>
__global__ __launch_bounds__(BLOCK) void gmsd_kernel(GmsdArgs a) {
  // one task per workgroup: its four waves take four adjacent strips over the
  // same rows, so each input row is fetched as one contiguous stretch
  const int task = static_cast<int>(xcd_tile(blockIdx.x, gridDim.x));
  if (task >= a.tasks) return;  // whole workgroup; no barrier follows
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int lane = threadIdx.x % WAVE;
  const int n = task / a.wpi;
  const int k = task - n * a.wpi;
  // this workgroup's share [s, e) of the image's (channel, group, row) space
  int64_t s = a.rows_img * k / a.wpi;
  const int64_t e = a.rows_img * (k + 1) / a.wpi;
  const int64_t per_plane = static_cast<int64_t>(a.groups) * a.Hout;
  double acc = 0.0, acc2 = 0.0;
  // Odd shares walk bottom-up, from their end: two neighbouring shares then
  // read the sample rows around their common boundary at the same time (both
  // at the start, or both at the end), on the same XCD (consecutive tasks
  // share one), so the second read of those halo rows is an L2 hit.
  if ((k & 1) == 0) {
    while (s < e) {  // uniform; one run per strip group touched
      const int c = static_cast<int>(s / per_plane);
      const int64_t rem = s - c * per_plane;
      const int grp = static_cast<int>(rem / a.Hout);
      const int row = static_cast<int>(rem - static_cast<int64_t>(grp) * a.Hout);
      const int len = static_cast<int>(min(e - s, static_cast<int64_t>(a.Hout - row)));
      const int strip = grp * WAVES_PER_BLOCK + wave;
      if (strip < a.strips) gmsd_run<Src, MAP>(a, n, c, strip, row, len, false, acc, acc2);
      s += len;
    }
  } else {
    int64_t t = e;
    while (t > s) {  // uniform; the runs in reverse order
      const int64_t q = t - 1;  // last row of the run
      const int c = static_cast<int>(q / per_plane);
      const int64_t rem = q - c * per_plane;
      const int grp = static_cast<int>(rem / a.Hout);
      const int rq = static_cast<int>(rem - static_cast<int64_t>(grp) * a.Hout);
      const int len = static_cast<int>(min(t - s, static_cast<int64_t>(rq + 1)));
      const int strip = grp * WAVES_PER_BLOCK + wave;
      if (strip < a.strips) gmsd_run<Src, MAP>(a, n, c, strip, rq - len + 1, len, true, acc, acc2);
      t -= len;
    }
  }
  acc = wave_sum(acc);
  acc2 = wave_sum(acc2);
  if constexpr (FIN) {
    // the workgroup's two sums, in wave order, then one lane per word
    __shared__ double s_f[2 * WAVES_PER_BLOCK];
    if (lane == 0) {
      s_f[wave] = acc;
      s_f[WAVES_PER_BLOCK + wave] = acc2;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
      double v = 0.0;
#pragma unroll
      for (int w = 0; w < WAVES_PER_BLOCK; ++w) v += s_f[threadIdx.x * WAVES_PER_BLOCK + w];
      gmsd_finish(a, n, static_cast<int>(threadIdx.x), v);
    }
  } else if (lane == 0) {
    const int slot = task * WAVES_PER_BLOCK + wave;
    a.psum[slot] = acc;
    a.psumsq[slot] = acc2;
  }
}

// Block b reduces image b: mean and population standard deviation of its map
// (reference fa_cuda.cu:1005-1026), from the sums of d = 1 - q.
// A NaN variance (a NaN q, e.g. a flat patch with T = eps = 0) stays NaN, as
// the reference's portable statistics give (functional.py:959-971); its
// CUDA finalize clamps it to 0 instead.  With out_batch, block N (one more)
// forms the batch means of both statistics from the per-image sums, in image
// order.
__global__ __launch_bounds__(BLOCK) void gmsd_finalize_kernel(
    const double* __restrict__ psum, const double* __restrict__ psumsq, int ncols,
    double npix, double* __restrict__ out_mean, double* __restrict__ out_std, int N,
    double* __restrict__ out_batch) {
  __shared__ double smem[2 * WAVES_PER_BLOCK];
  const bool batch = static_cast<int>(blockIdx.x) == N;
  double bm = 0.0, bs = 0.0;
  for (int img = batch ? 0 : blockIdx.x; img < (batch ? N : static_cast<int>(blockIdx.x) + 1);
       ++img) {  // uniform
    const int64_t base = static_cast<int64_t>(img) * ncols;
    double a = 0.0, b = 0.0;
    for (int i = threadIdx.x; i < ncols; i += BLOCK) {
      a += psum[base + i];
      b += psumsq[base + i];
    }
    double sa = 0.0, sb = 0.0;
    block_sum2(a, b, smem, &sa, &sb);
    __syncthreads();  // smem is reused by the next image
    if (threadIdx.x == 0) {
      double m, sd;
      gmsd_stats(sa, sb, npix, &m, &sd);
      if (batch) {
        bm += m;
        bs += sd;
      } else {
        out_mean[img] = m;
        out_std[img] = sd;
      }
    }
  }
  if (batch && threadIdx.x == 0) {
    out_batch[0] = bm / N;
    out_batch[1] = bs / N;
  }
}

// --------------------------------------------------------------------------
// backward (an extension): gradients of per-image mean and standard
// deviation of q, for x / y of float32 or float64, all in float64.
//
//   coefficient pass: per output pixel, with w = dL/dq = g_mean/n +
//     g_std (q - m)/(n std), dq/dg1 = 2 (g2 - g1)(g2 (g1 + g2) + T)/D^2 (the
//     factored form, exact in sign and accurate where g1 ~ g2) and
//     dg/dgx = gx/g: the four maps dL/dgx1, dL/dgy1, dL/dgx2, dL/dgy2.
//     A workgroup stages the (16 + 2) x (64 + 2) samples of its tile in LDS.
//   scatter: per input pixel, the Prewitt adjoint of those maps at its
//     sample (12 taps per tensor, zero outside the map), a quarter of it with
//     downsampling, none for the dropped odd row / column.
// --------------------------------------------------------------------------
constexpr int GB_TR = 16;  // output rows per coefficient tile
constexpr int GB_TC = 64;  // output columns per coefficient tile

struct GmsdBwdArgs {
  const void* x;
  const void* y;
  int C, H, W, Hd, Wd, Hout, Wout;
  double T, eps;
  const double* mean;
  const double* std_;
  const double* g_mean;  // may be null: zero
  const double* g_std;   // may be null: zero
  double* aux;           // 4 maps [planes, Hout, Wout]
  int64_t map_stride;    // planes * Hout * Wout
  void* dx;
  void* dy;
  int tiles_x, tiles_y;
};

template <typename T, bool DOWN>
__device__ inline double gb_sample(const T* plane, int W, int r, int c) {
  if constexpr (DOWN) {
    const int64_t o = static_cast<int64_t>(2 * r) * W + 2 * c;
    return 0.25 * ((Elem<T>::d(plane[o]) + Elem<T>::d(plane[o + 1])) +
                   (Elem<T>::d(plane[o + W]) + Elem<T>::d(plane[o + W + 1])));
  } else {
    return Elem<T>::d(plane[static_cast<int64_t>(r) * W + c]);
  }
}

template <typename T, bool DOWN>
__global__ __launch_bounds__(BLOCK) void gmsd_coef_kernel(GmsdBwdArgs a) {
  __shared__ double sx[GB_TR + 2][GB_TC + 2];
  __shared__ double sy[GB_TR + 2][GB_TC + 2];
  const int per_plane = a.tiles_x * a.tiles_y;
  const int plane = blockIdx.x / per_plane;
  const int t = blockIdx.x - plane * per_plane;
  const int R0 = (t / a.tiles_x) * GB_TR;
  const int C0 = (t % a.tiles_x) * GB_TC;
  const int64_t poff = static_cast<int64_t>(plane) * a.H * a.W;
  const T* px = static_cast<const T*>(a.x) + poff;
  const T* py = static_cast<const T*>(a.y) + poff;
  // stage the samples; rows / columns past the sample grid are clamped (they
  // only feed outputs outside the map)
  for (int e = threadIdx.x; e < (GB_TR + 2) * (GB_TC + 2); e += BLOCK) {
    const int r = e / (GB_TC + 2), c = e - r * (GB_TC + 2);
    const int gr = min(R0 + r, a.Hd - 1), gc = min(C0 + c, a.Wd - 1);
    sx[r][c] = gb_sample<T, DOWN>(px, a.W, gr, gc);
    sy[r][c] = gb_sample<T, DOWN>(py, a.W, gr, gc);
  }
  __syncthreads();

  const int n = plane / a.C;
  const double cnt = static_cast<double>(a.C) * a.Hout * a.Wout;
  const double gm = a.g_mean ? a.g_mean[n] : 0.0;
  const double gsd = a.g_std ? a.g_std[n] : 0.0;
  const double sd = a.std_[n];
  const double ks = sd > 0.0 ? gsd / (cnt * sd) : 0.0;
  const double m = a.mean[n];
  const double third = 1.0 / 3.0;
  for (int e = threadIdx.x; e < GB_TR * GB_TC; e += BLOCK) {
    const int i = e / GB_TC, j = e - i * GB_TC;
    const int oi = R0 + i, oj = C0 + j;
    if (oi >= a.Hout || oj >= a.Wout) continue;
    double gx1 = 0.0, gy1 = 0.0, gx2 = 0.0, gy2 = 0.0;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      gx1 += sx[i + u][j] - sx[i + u][j + 2];
      gy1 += sx[i][j + u] - sx[i + 2][j + u];
      gx2 += sy[i + u][j] - sy[i + u][j + 2];
      gy2 += sy[i][j + u] - sy[i + 2][j + u];
    }
    gx1 *= third;
    gy1 *= third;
    gx2 *= third;
    gy2 *= third;
    const double G1 = fma(gx1, gx1, fma(gy1, gy1, a.eps));
    const double G2 = fma(gx2, gx2, fma(gy2, gy2, a.eps));
    const double g1 = sqrt(G1), g2 = sqrt(G2);
    const double D = G1 + G2 + a.T;
    const double q = fma(2.0 * g1, g2, a.T) / D;
    const double w = gm / cnt + ks * (q - m);
    // g2 - g1 = (G2 - G1) / (g1 + g2), with G2 - G1 in factored form
    const double dG = fma(gx2 - gx1, gx2 + gx1, (gy2 - gy1) * (gy2 + gy1));
    const double dg = dG / (g1 + g2);
    const double iD2 = 1.0 / (D * D);
    const double d1 = w * 2.0 * dg * fma(g2, g1 + g2, a.T) * iD2;   // w dq/dg1
    const double d2 = -w * 2.0 * dg * fma(g1, g1 + g2, a.T) * iD2;  // w dq/dg2
    const int64_t o = static_cast<int64_t>(plane) * a.Hout * a.Wout +
                      static_cast<int64_t>(oi) * a.Wout + oj;
    a.aux[o] = d1 * gx1 / g1;
    a.aux[a.map_stride + o] = d1 * gy1 / g1;
    a.aux[2 * a.map_stride + o] = d2 * gx2 / g2;
    a.aux[3 * a.map_stride + o] = d2 * gy2 / g2;
  }
}

// (1/3) sum_u [Gx(a-u, b) - Gx(a-u, b-2)] + (1/3) sum_u [Gy(a, b-u) - Gy(a-2, b-u)]
__device__ inline double prewitt_adjoint(const double* gx, const double* gy, int Hout, int Wout,
                                         int r, int c) {
  auto at = [&](const double* m, int i, int j) {
    return (i >= 0 && i < Hout && j >= 0 && j < Wout) ? m[static_cast<int64_t>(i) * Wout + j]
                                                      : 0.0;
  };
  double s = 0.0;
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    s += at(gx, r - u, c) - at(gx, r - u, c - 2);
    s += at(gy, r, c - u) - at(gy, r - 2, c - u);
  }
  return s * (1.0 / 3.0);
}

template <typename T, bool DOWN>
__global__ __launch_bounds__(BLOCK) void gmsd_scatter_kernel(GmsdBwdArgs a, int64_t total) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * BLOCK + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * BLOCK) {
    const int64_t plane = e / (static_cast<int64_t>(a.H) * a.W);
    const int64_t rem = e - plane * a.H * a.W;
    const int h = static_cast<int>(rem / a.W), w = static_cast<int>(rem - (rem / a.W) * a.W);
    const int r = DOWN ? h / 2 : h, c = DOWN ? w / 2 : w;
    const bool in = r < a.Hd && c < a.Wd;  // the dropped odd row / column
    const int64_t mo = plane * a.Hout * a.Wout;
    const double scale = DOWN ? 0.25 : 1.0;
    if (a.dx) {
      const double v = in ? scale * prewitt_adjoint(a.aux + mo, a.aux + a.map_stride + mo,
                                                    a.Hout, a.Wout, r, c)
                          : 0.0;
      static_cast<T*>(a.dx)[e] = static_cast<T>(v);
    }
    if (a.dy) {
      const double v = in ? scale * prewitt_adjoint(a.aux + 2 * a.map_stride + mo,
                                                    a.aux + 3 * a.map_stride + mo, a.Hout,
                                                    a.Wout, r, c)
                          : 0.0;
      static_cast<T*>(a.dy)[e] = static_cast<T>(v);
    }
  }
}

template <typename T, bool DOWN>
static int launch_gmsd_bwd(GmsdBwdArgs& a, int64_t planes, int device, hipStream_t st) {
  a.tiles_x = (a.Wout + GB_TC - 1) / GB_TC;
  a.tiles_y = (a.Hout + GB_TR - 1) / GB_TR;
  const int64_t wgs = planes * a.tiles_x * a.tiles_y;
  if (wgs > INT32_MAX) return FA_E_SHAPE;
  hipLaunchKernelGGL((gmsd_coef_kernel<T, DOWN>), dim3(static_cast<unsigned>(wgs)), dim3(BLOCK),
                     0, st, a);
  FA_LAUNCH_CHECK();
  const int64_t total = planes * a.H * a.W;
  const int64_t want = (total + BLOCK - 1) / BLOCK;
  const int64_t cap = static_cast<int64_t>(cu_count(device)) * 16;
  hipLaunchKernelGGL((gmsd_scatter_kernel<T, DOWN>),
                     dim3(static_cast<unsigned>(want < cap ? want : cap)), dim3(BLOCK), 0, st, a,
                     total);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

struct GGeom {
  int Hd, Wd, Hout, Wout;
};

static int gmsd_geometry(int H, int W, int downsample, GGeom* g) {
  if (H <= 0 || W <= 0) return FA_E_SHAPE;
  g->Hd = downsample ? H / 2 : H;
  g->Wd = downsample ? W / 2 : W;
  g->Hout = g->Hd - 2;
  g->Wout = g->Wd - 2;
  if (g->Hout <= 0 || g->Wout <= 0) return FA_E_SHAPE;
  return FA_OK;
}

// Partial slots per output plane (the workspace query): one per G_SLOT_ROWS
// rows of the narrowest strips, and at least one workgroup's worth.  A launch
// uses at most Cout * slots per image, one per wave.
static int gmsd_slots(const GGeom& g) {
  const int strips = (g.Wout + G_OUTW_NARROW - 1) / G_OUTW_NARROW;
  const int chunks = (g.Hout + G_SLOT_ROWS - 1) / G_SLOT_ROWS;
  return std::max(strips * chunks, WAVES_PER_BLOCK);
}

static bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

template <class Src, bool MAP, bool FIN = false>
static int occupancy_gmsd() {
  static int wgs_per_cu = 0;  // occupancy of this kernel, queried once
  if (wgs_per_cu <= 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &v, reinterpret_cast<const void*>(&gmsd_kernel<Src, MAP, FIN>), BLOCK, 0) != hipSuccess ||
        v <= 0)
      v = 1;
    wgs_per_cu = v;
  }
  return wgs_per_cu;
}

// Workgroups per image: one round of resident workgroups over the whole
// launch, no more than the workspace holds (a slot per wave) or than leaves a
// workgroup G_MIN_ROWS rows.  The kernel that writes the q map is its own
// instantiation, so the statistics-only one carries no map test.  With
// a.acc set (and no map) the launch finishes the call itself when its
// workgroups per image fit the finish's count bits: *wpi_used is then 0.
template <class Src>
static int launch_gmsd(GmsdArgs a, int N, int slots_per_image, int device, hipStream_t st,
                       int* wpi_used) {
  const bool map = a.map != nullptr;
  const bool fin_ok = a.acc && !map;
  // a workgroup is one wave on each of the CU's four SIMDs
  const int wgs_per_cu = std::min(
      G_MAX_WAVES_PER_SIMD, map ? occupancy_gmsd<Src, true>()
                                : (fin_ok ? occupancy_gmsd<Src, false, true>()
                                          : occupancy_gmsd<Src, false>()));
  a.strips = (a.Wout + Src::OUTW - 1) / Src::OUTW;
  a.groups = (a.strips + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  a.rows_img = static_cast<int64_t>(a.Cout) * a.groups * a.Hout;
  const int64_t resident = static_cast<int64_t>(cu_count(device)) * wgs_per_cu;
  int64_t wpi = (resident + N - 1) / N;
  wpi = std::min<int64_t>(wpi, (a.rows_img + G_MIN_ROWS - 1) / G_MIN_ROWS);
  wpi = std::min<int64_t>(wpi, slots_per_image / WAVES_PER_BLOCK);
  wpi = std::max<int64_t>(wpi, 1);
  const int64_t tasks = static_cast<int64_t>(N) * wpi;
  if (tasks > INT32_MAX / WAVES_PER_BLOCK) return FA_E_SHAPE;
  a.wpi = static_cast<int>(wpi);
  a.tasks = static_cast<int>(tasks);
  if ((!a.psum || !a.psumsq) && !(fin_ok && wpi < (1 << GF_COUNT_BITS))) return FA_E_ARG;
  if (fin_ok && wpi < (1 << GF_COUNT_BITS)) {
    hipLaunchKernelGGL((gmsd_kernel<Src, false, true>), dim3(static_cast<unsigned>(tasks)),
                       dim3(BLOCK), 0, st, a);
    FA_LAUNCH_CHECK();
    *wpi_used = 0;
    return FA_OK;
  }
  if (map)
    hipLaunchKernelGGL((gmsd_kernel<Src, true>), dim3(static_cast<unsigned>(tasks)), dim3(BLOCK),
                       0, st, a);
  else
    hipLaunchKernelGGL((gmsd_kernel<Src, false>), dim3(static_cast<unsigned>(tasks)), dim3(BLOCK),
                       0, st, a);
  FA_LAUNCH_CHECK();
  *wpi_used = a.wpi * WAVES_PER_BLOCK;  // partial slots per image
  return FA_OK;
}

struct GLaunch {
  int N, slots, device;
  hipStream_t st;
};

template <typename T, bool LUMA>
static int dispatch_gmsd_t(const GmsdArgs& a, const GLaunch& l, bool down, int* wpi) {
  if (down) return launch_gmsd<SrcGeneric<T, true, LUMA>>(a, l.N, l.slots, l.device, l.st, wpi);
  return launch_gmsd<SrcGeneric<T, false, LUMA>>(a, l.N, l.slots, l.device, l.st, wpi);
}

template <bool LUMA>
static int dispatch_gmsd(int dtype, const GmsdArgs& a, const GLaunch& l, bool down, bool wide,
                         int* wpi) {
  switch (dtype) {
    case FA_U8:
      if (wide) return launch_gmsd<SrcU8Wide<LUMA>>(a, l.N, l.slots, l.device, l.st, wpi);
      return dispatch_gmsd_t<uint8_t, LUMA>(a, l, down, wpi);
    case FA_F16: return dispatch_gmsd_t<half_t, LUMA>(a, l, down, wpi);
    case FA_BF16: return dispatch_gmsd_t<bf16_t, LUMA>(a, l, down, wpi);
    case FA_F32: return dispatch_gmsd_t<float, LUMA>(a, l, down, wpi);
    case FA_F64: return dispatch_gmsd_t<double, LUMA>(a, l, down, wpi);
    default: return FA_E_DTYPE;
  }
}

static int gmsd_impl(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                     const int64_t* xs, const int64_t* ys, const double* luma, double Tc,
                     double eps, int downsample, float* map_out, double* psum, double* psumsq,
                     int bpp, double* out_mean, double* out_std, int device, void* stream,
                     uint64_t* acc = nullptr, double* out_batch = nullptr) {
  // null psum / psumsq are enough only where the launch finishes the call
  // (launch_gmsd refuses them otherwise, before launching)
  if (!x || !y || !out_mean || !out_std) return FA_E_ARG;
  if ((!psum || !psumsq) && !acc) return FA_E_ARG;
  if (N <= 0 || C <= 0) return FA_E_SHAPE;
  if (dtype < FA_U8 || dtype > FA_F64) return FA_E_DTYPE;
  if (luma && C != 3) return FA_E_SHAPE;
  GGeom g;
  const int rc = gmsd_geometry(H, W, downsample, &g);
  if (rc != FA_OK) return rc;
  if (bpp != gmsd_slots(g)) return FA_E_ARG;

  GmsdArgs a = {};
  a.x = x;
  a.y = y;
  const int64_t cs = static_cast<int64_t>(H) * W;
  a.vx = xs ? GView{xs[0], xs[1], xs[2]} : GView{cs * C, cs, W};
  a.vy = ys ? GView{ys[0], ys[1], ys[2]} : GView{cs * C, cs, W};
  // rows may not overlap; planes and images run forward
  if (a.vx.sh < W || a.vy.sh < W || a.vx.sc < 0 || a.vy.sc < 0 || a.vx.sn < 0 || a.vy.sn < 0)
    return FA_E_SHAPE;
  a.Cout = luma ? 1 : C;
  a.Hd = g.Hd;
  a.Wd = g.Wd;
  a.Hout = g.Hout;
  a.Wout = g.Wout;
  if (luma) {
    a.kr = luma[0];
    a.kg = luma[1];
    a.kb = luma[2];
  }
  const double sc2 = downsample ? 144.0 : 9.0;  // 9 s^2
  a.T2 = Tc * sc2;
  a.eps2 = eps * sc2;
  // The float32 path's denominators stay positive when eps or T is positive
  // and at least 1e-18 (see one_minus_q), so positive values below 1e-18 are
  // raised to it: the defaults are far above, and adding 1e-18 to G = gx^2 +
  // gy^2 + eps moves a term by at most ~1e-9 relative even where G is tiny.
  // Zero stays zero: with T = eps = 0 a flat pixel is 0 / 0 = NaN, as in the
  // reference (fa_cuda.cu:987-988, functional.py:950-956).
  const auto floor18 = [](double v) { return static_cast<float>(v > 0.0 && v < 1e-18 ? 1e-18 : v); };
  a.T2f = floor18(a.T2);
  a.eps2f = floor18(a.eps2);
  a.psum = psum;
  a.psumsq = psumsq;
  a.map = map_out;
  // the one-launch finish: T or eps positive (the d of finite samples in
  // [0, 1]; NaN and inf samples flag their image, see gmsd_finish), statistics
  // only, at most GF_MAX_IMAGES images; the fixed-point scale leaves a sum of d
  // (or d^2) over the image, each at most 1 (plus float32 rounding), below
  // 2^(64 - GF_COUNT_BITS)
  const double npix = static_cast<double>(g.Hout) * g.Wout * a.Cout;
  if (acc && !map_out && N <= GF_MAX_IMAGES && (a.T2f > 0.0f || a.eps2f > 0.0f)) {
    int bits = 1;
    while (bits < 40 && std::ldexp(1.0, bits) <= 2.0 * npix) ++bits;
    if (bits < 40) {
      a.acc = acc;
      a.fscale = std::ldexp(1.0, 64 - GF_COUNT_BITS - bits);
      a.finv = std::ldexp(1.0, bits - (64 - GF_COUNT_BITS));
      a.npix = npix;
      a.out_mean = out_mean;
      a.out_std = out_std;
      a.out_batch = out_batch;
      a.N = N;
    }
  }
  const bool down = downsample != 0;
  // the dword path: uint8, downsampled, every row of every plane 4-byte aligned
  // (buffer addressing: a plane's rows must lie within 2^31 bytes of its base)
  const int64_t ext_x = static_cast<int64_t>(2 * g.Hd - 1) * a.vx.sh + W;
  const int64_t ext_y = static_cast<int64_t>(2 * g.Hd - 1) * a.vy.sh + W;
  const int64_t strides = a.vx.sn | a.vx.sc | a.vx.sh | a.vy.sn | a.vy.sc | a.vy.sh;
  const bool wide = dtype == FA_U8 && down && W % 4 == 0 && aligned4(x) && aligned4(y) &&
                    (strides & 3) == 0 && ext_x <= INT32_MAX && ext_y <= INT32_MAX;
  a.ext_x = wide ? static_cast<int>(ext_x) : 0;
  a.ext_y = wide ? static_cast<int>(ext_y) : 0;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const GLaunch l = {N, a.Cout * bpp, device, st};  // psum is [N * Cout, bpp]
  int wpi = 0;
  const int r = luma ? dispatch_gmsd<true>(dtype, a, l, down, wide, &wpi)
                     : dispatch_gmsd<false>(dtype, a, l, down, wide, &wpi);
  if (r != FA_OK) return r;
  if (wpi == 0) return FA_OK;  // finished inside the launch
  // each image owns wpi consecutive slots, one per wave
  hipLaunchKernelGGL(gmsd_finalize_kernel, dim3(static_cast<unsigned>(N + (out_batch ? 1 : 0))),
                     dim3(BLOCK), 0, st, psum, psumsq, wpi, npix, out_mean, out_std, N,
                     out_batch);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

}  // namespace fa

using namespace fa;

extern "C" {

// reference: fa_cuda.cu:1416-1424 (fa_cuda_gmsd_workspace)
FA_API int fa_gpu_gmsd_workspace(int H, int W, int downsample, int* out_bpp) {
  if (!out_bpp) return FA_E_ARG;
  GGeom g;
  const int rc = gmsd_geometry(H, W, downsample, &g);
  if (rc != FA_OK) return rc;
  *out_bpp = gmsd_slots(g);
  return FA_OK;
}

// reference: fa_cuda.cu:1426-1466 (fa_cuda_gmsd)
FA_API int fa_gpu_gmsd(const void* x, const void* y, int dtype, int N, int C,
                       int H, int W, double Tc, double eps, int downsample,
                       double* psum, double* psumsq, int bpp, double* out_mean,
                       double* out_std, int device, void* stream) {
  return gmsd_impl(x, y, dtype, N, C, H, W, nullptr, nullptr, nullptr, Tc, eps, downsample,
                   nullptr, psum, psumsq, bpp, out_mean, out_std, device, stream);
}

// No counterpart in the reference, which materialises a float32 luma plane
// (functional.py:267-271) and copies crops contiguous (backend.py:346,482).
FA_API int fa_gpu_gmsd_ex(const void* x, const void* y, int dtype, int N, int C,
                          int H, int W, const int64_t* x_strides,
                          const int64_t* y_strides, const double* luma, double Tc,
                          double eps, int downsample, float* map_out, double* psum,
                          double* psumsq, int bpp, double* out_mean, double* out_std,
                          int device, void* stream) {
  return gmsd_impl(x, y, dtype, N, C, H, W, x_strides, y_strides, luma, Tc, eps, downsample,
                   map_out, psum, psumsq, bpp, out_mean, out_std, device, stream);
}

// No counterpart in the reference, whose GMSD ends in a finalize launch
// (fa_cuda.cu:1460-1465) and takes batch means with torch (functional.py:1082):
// fa_gpu_gmsd_ex without the map, finished inside the launch where it can be.
FA_API int fa_gpu_gmsd_once(const void* x, const void* y, int dtype, int N, int C, int H,
                            int W, const int64_t* x_strides, const int64_t* y_strides,
                            const double* luma, double Tc, double eps, int downsample,
                            double* psum, double* psumsq, int bpp, uint64_t* acc,
                            double* out_mean, double* out_std, double* out_batch, int device,
                            void* stream) {
  return gmsd_impl(x, y, dtype, N, C, H, W, x_strides, y_strides, luma, Tc, eps, downsample,
                   nullptr, psum, psumsq, bpp, out_mean, out_std, device, stream, acc,
                   out_batch);
}

// No counterpart in the reference: its GMS / GMSD losses differentiate the
// portable PyTorch path (modules.py:183-184).  Gradients of
//   L = sum_n g_mean[n] mean_n(q) + g_std[n] std_n(q)
// with respect to contiguous x and y (N x C x H x W, FA_F32 or FA_F64); mean /
// std are fa_gpu_gmsd's outputs for the same inputs; g_mean / g_std are
// device arrays of N (either may be null: zero); aux is 4 * N*C*Hout*Wout
// float64 scratch; dx / dy (either may be null) are written in full.
FA_API int fa_gpu_gmsd_backward(const void* x, const void* y, int dtype, int N, int C, int H,
                                int W, double Tc, double eps, int downsample,
                                const double* mean, const double* std_dev,
                                const double* g_mean, const double* g_std, double* aux,
                                void* dx, void* dy, int device, void* stream) {
  if (!x || !y || !mean || !std_dev || !aux) return FA_E_ARG;
  if (!dx && !dy) return FA_E_ARG;
  if (dtype != FA_F32 && dtype != FA_F64) return FA_E_DTYPE;
  if (N <= 0 || C <= 0) return FA_E_SHAPE;
  GGeom g;
  const int rc = gmsd_geometry(H, W, downsample, &g);
  if (rc != FA_OK) return rc;
  GmsdBwdArgs a = {};
  a.x = x;
  a.y = y;
  a.C = C;
  a.H = H;
  a.W = W;
  a.Hd = g.Hd;
  a.Wd = g.Wd;
  a.Hout = g.Hout;
  a.Wout = g.Wout;
  a.T = Tc;
  a.eps = eps;
  a.mean = mean;
  a.std_ = std_dev;
  a.g_mean = g_mean;
  a.g_std = g_std;
  a.aux = aux;
  const int64_t planes = static_cast<int64_t>(N) * C;
  a.map_stride = planes * g.Hout * g.Wout;
  a.dx = dx;
  a.dy = dy;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool down = downsample != 0;
  if (dtype == FA_F32)
    return down ? launch_gmsd_bwd<float, true>(a, planes, device, st)
                : launch_gmsd_bwd<float, false>(a, planes, device, st);
  return down ? launch_gmsd_bwd<double, true>(a, planes, device, st)
              : launch_gmsd_bwd<double, false>(a, planes, device, st);
}

}  // extern "C"
