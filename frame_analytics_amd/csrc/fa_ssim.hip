// SSIM family on gfx950: forward (mean / per-image / map), the MS-SSIM
// per-scale primitive (SSIM and cs plane means), and the analytic backward.
//
// Semantics follow the reference (fa_cuda.cu:389-784, 1158-1414):
//   * inputs are shifted by `shift` (= L/2) before filtering; the shift cancels
//     out of every variance term and is added back to the means
//   * four blurred moment planes x', y', x'y', (x'-y')^2 -- sigma_x^2+sigma_y^2
//     is recovered as E[(x'-y')^2] + 2 sigma_xy - (mu_x - mu_y)^2, which keeps
//     every intermediate the size of the answer
//   * SSIM = (2 mu_x mu_y + C1)(2 sigma_xy + C2) / ((mu_x^2+mu_y^2+C1)(sigma_x^2+sigma_y^2+C2))
//   * cs = (2 sigma_xy + C2) / (sigma_x^2 + sigma_y^2 + C2)
//   * backward: per output pixel b = g dS/dsigma_xx, c = g dS/dsigma_xy,
//     t_x = g dS/dmu_x - 2 b mu_x' - c mu_y'; then
//     dx = 2 x' (w * b) + y' (w * c) + (w * t_x) on the full grid.
//
// The MI355X-specific choices:
//   * every kernel is the register-ring / LDS strip engine of fa_strip.h
//   * the backward computes in float64 throughout (moments, coefficients,
//     scatter): CDNA4 retires FP64 FMA at the unpacked FP32 rate, so exact-ish
//     gradients cost registers, not time.  Only the aux maps and dx are stored
//     as float32, as the C ABI prescribes.
//   * float64 inputs get a float64 forward instead of a refusal.
//   * the block partial sums are float64 and reduced in a fixed order.
#include "fa_strip.h"
#include "fa_ssim_mfma.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace fa {

// MODE_CSF: the CS pass of a training step, in float64, which also writes
// the coefficient maps of MODE_PREP_CS for a unit gradient of one plane mean
// (the SSIM means or the cs means, SsimArgs::unit_s): MS-SSIM's loss reads
// only one of them at each scale, so the maps the backward needs are these
// times that plane's upstream gradient, and no coefficient pass runs there.
enum { MODE_REDUCE = 0, MODE_MAP = 1, MODE_CS = 2, MODE_PREP = 3, MODE_PREP_CS = 4,
       MODE_CSF = 5 };

// Output rows per workgroup (TH), a multiple of 4 up to 128.  A workgroup
// walks its rows in sequence and re-reads K-1 halo rows, so a launch trades
// rounds of resident workgroups against rows per workgroup (tiling_for):
// configs of many large frames take long chunks (configs[1]: TH = 68, 3072
// workgroups = 3 rounds of 1024), while single frames,
// the coarse MS-SSIM scales and small crops get the parallelism back, and the
// float64 backward kernels (one workgroup per CU) are cut only as fine as
// they can use.  Every TH is a multiple of the phase height and even, so
// pyramid row pairs never straddle two chunks.  The partial buffers are
// sized for the smallest TH (the *_workspace queries) and a launch uses the
// first strips * chunks slots of each plane.
#ifndef FA_SSIM_TH_MAX
#define FA_SSIM_TH_MAX 128
#endif
constexpr int SSIM_TH_MAX = FA_SSIM_TH_MAX;
constexpr int SSIM_TH_MIN = 4;
constexpr int SSIM_TH_STEP = 4;
static_assert(SSIM_TH_MIN % PH == 0 && SSIM_TH_STEP % PH == 0 && SSIM_TH_MAX % SSIM_TH_STEP == 0,
              "TH ladder");

struct Tiling {
  int TH, strips, tiles;  // tiles = strips * chunks, per plane
};

// The tiling of one launch over `planes` planes of an out_H x out_W grid
// when the chip holds `resident` workgroups at once: the TH that minimises
// rounds x work per workgroup, ceil(wgs / resident) * (TH + (K + 1) / 2),
// in output rows; ties keep the larger TH.  A halo row only forms its
// moments, so the K - 1 halo rows and the set-up weigh about half as much as
// the output rows.  Measured on MI355X (TH any multiple of 4 up to 128):
//                           charged TH+K+1   TH+(K+1)/2   (64/32/16/8/4, TH+K+1)
//   configs[1] kernel         156.7 us        147.4         147.6
//   1x3x1080x1920 call         27.6            27.6          30.4
//   MS-SSIM configs[4] call   274.4           264.4         264.5
//   MS-SSIM loss step        1887            1848          1920
// (Charging a partial round only its share was measured slower: MS-SSIM
// 301 vs 291 us, the float64 backward 155 vs 133 us.)
inline Tiling tiling_for(int64_t planes, int out_H, int out_W, int K, int64_t resident) {
  Tiling best = {0, 0, 0};
  int64_t best_cost = INT64_MAX;
  for (int th = SSIM_TH_MAX; th >= SSIM_TH_MIN; th -= SSIM_TH_STEP) {
    int strips = 0, chunks = 0;
    strip_grid(out_H, out_W, K, th, &strips, &chunks);
    const int64_t wgs = planes * strips * chunks;
    const int64_t cost = ((wgs + resident - 1) / resident) * (th + (K + 1) / 2);
    if (cost < best_cost) {
      best_cost = cost;
      best = Tiling{th, strips, strips * chunks};
    }
  }
  return best;
}

// Partial slots per plane the workspace query reports: enough for any TH.
inline int ssim_slots(int out_H, int out_W, int K) {
  int strips = 0, chunks = 0;
  strip_grid(out_H, out_W, K, SSIM_TH_MIN, &strips, &chunks);
  return strips * chunks;
}

// a / b.  The float32 forward uses v_rcp_f32 (1 ulp) and a multiply instead of
// the ~9-instruction IEEE division sequence; float64 divides exactly.
__device__ inline float quot(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }
__device__ inline double quot(double a, double b) { return a / b; }

struct SsimArgs {
  const void* x;
  const void* y;
  int H, W, Hout, Wout, TH, strips, bpp;
  double shift, C1, C2;
  const float* win;
  float* map;           // MODE_MAP
  double* partial;      // MODE_REDUCE / MAP / CS
  SsimFin fin;          // MODE_REDUCE: with fin.acc, the one-launch finish
                        //   (ssim_fin_add) in place of the partial slots
  double* partial_cs;   // MODE_CS
  const float* dmap;    // MODE_PREP: full upstream map, or null
  const float* gscalar; // MODE_PREP: device scalar used when dmap is null
  double gnorm;         // MODE_PREP(_CS): 1/(npix*planes) or 1/npix
  const float* gs;      // MODE_PREP_CS: per-plane dL/d(mean ssim)
  const float* gcs;     // MODE_PREP_CS: per-plane dL/d(mean cs)
  int unit_s;           // MODE_CSF: maps for d(mean ssim) = 1 (1) or d(mean cs) = 1 (0)
  float* ob;
  float* oc;
  float* otx;
  float* oty;
  void* px;             // MODE_CS: optional pyramid step (2x2 means of x / y)
  void* py;
  int pool_f64;         // pyramid element type: float64 (1) or float32 (0),
  int pool_f16;         //   or float16 (uint8 input without luma only)
  // input views (forward modes): element strides of image and channel, row
  // stride; columns are contiguous.  Planes are (image, output channel).
  int64_t xsn, xsc, ysn, ysc;
  int xsh, ysh;
  int Cout;             // output planes per image (1 with luma)
  double kr, kg, kb;    // luma weights
  double offset;        // luma offset: added to every sample the kernel forms
};

template <typename T, typename CTy, int MODE, bool LUMA = false>
struct SsimPol {
  static constexpr int NP = 4;
  static constexpr int CH = LUMA ? 3 : 1;
  using CT = CTy;
  struct Raw {
    CT x, y;
  };
  // Ring rows: the four moments at float32; at float64 only x', y', whose
  // products vtap forms per tap (exact in float64, so the sums are the same
  // bits) -- half the ring's registers.
  using RT = CT;
  static constexpr int NR = sizeof(CT) == 8 ? 2 : 4;

  const T* __restrict__ x[CH];  // this plane of x (the R, G, B planes with luma)
  const T* __restrict__ y[CH];
  int H, W;
  uint32_t shx, shy;        // row strides
  uint32_t lcol;            // this lane's column, clamped into the image
  CT kr, kg, kb;            // luma weights
  CT cshift;                // shift - offset: centres the samples as loaded
  double poff;              // offset, added to the pyramid means
  CT shift, C1, C2;
  int64_t out_off;
  int Wout;
  float* __restrict__ map;
  float* __restrict__ ob;
  float* __restrict__ oc;
  float* __restrict__ otx;
  float* __restrict__ oty;
  const float* __restrict__ dmap;
  CT g_uniform, gS, gCS;
  CT k1;  // 2 shift^2 + C1
  CT row_s, row_cs;
  double acc_s, acc_cs;
  // MODE_CS pyramid step: this workgroup owns input rows [prow0, prow1) and,
  // on even lanes, the column pair starting at its column (pcol = col / 2)
  void* px;
  void* py;
  bool pool_on, pool_f64, pool_f16, pcol_ok;
  int prow0, prow1, Wd;
  int64_t pool_off;
  uint32_t pcol;
  // pyramid sums: a 2x2 block of uint8 sums to at most 1020, exact in
  // float32 (as is its quarter); every other input sums in float64
  using PA = typename std::conditional<std::is_same<T, uint8_t>::value && !LUMA, float,
                                       double>::type;

  // The forward's tap origin is 0, so rows and columns are never negative.
  // Rows past H and columns past W only feed outputs outside the map, so they
  // are clamped into the image instead of branched around.
  __device__ inline void set_column(int col) {
    lcol = static_cast<uint32_t>(col < W ? col : W - 1);
  }

  __device__ inline CT elem(const T* p, uint32_t o) const {
    if constexpr (sizeof(CT) == 8) return Elem<T>::d(p[o]);
    else return Elem<T>::f(p[o]);
  }

  __device__ inline Raw load(int row) const {
    // a plane spans < 2^31 elements (checked on the host): 32-bit offsets
    const uint32_t r = static_cast<uint32_t>(row < H ? row : H - 1);
    const uint32_t ox = r * shx + lcol, oy = r * shy + lcol;
    if constexpr (LUMA)
      return Raw{fma(kb, elem(x[2], ox), fma(kg, elem(x[1], ox), kr * elem(x[0], ox))),
                 fma(kb, elem(y[2], oy), fma(kg, elem(y[1], oy), kr * elem(y[0], oy)))};
    else
      return Raw{elem(x[0], ox), elem(y[0], oy)};
  }

  // The 2x2 means of rows (row, row + 1), row even, and columns (2j, 2j+1),
  // summed in PA (exact for the pyramid's element types) and written by the
  // even lane.  The engine hands both rows of a pair at once, so there is no
  // row-parity branch and no state between calls.
  __device__ inline void pool2(int row, const Raw& a, const Raw& b) {
    if constexpr (MODE == MODE_CS || MODE == MODE_CSF) {
      // prow1 is even, so row < prow1 covers row + 1 too
      if (!pool_on || row < prow0 || row >= prow1) return;  // uniform
      PA sx = static_cast<PA>(a.x) + static_cast<PA>(b.x);
      PA sy = static_cast<PA>(a.y) + static_cast<PA>(b.y);
      sx += lane_xor1(sx);
      sy += lane_xor1(sy);
      if (pcol_ok) {
        const int64_t o = pool_off + static_cast<int64_t>(row >> 1) * Wd + pcol;
        if (pool_f64) {
          static_cast<double*>(px)[o] = fma(0.25, static_cast<double>(sx), poff);
          static_cast<double*>(py)[o] = fma(0.25, static_cast<double>(sy), poff);
        } else if constexpr (std::is_same<PA, float>::value) {
          // poff is 0 without luma; a quarter of a byte sum is exact in float16
          if (pool_f16) {
            static_cast<_Float16*>(px)[o] = static_cast<_Float16>(PA(0.25) * sx);
            static_cast<_Float16*>(py)[o] = static_cast<_Float16>(PA(0.25) * sy);
          } else {
            static_cast<float*>(px)[o] = PA(0.25) * sx;
            static_cast<float*>(py)[o] = PA(0.25) * sy;
          }
        } else {
          static_cast<float*>(px)[o] = static_cast<float>(fma(0.25, sx, poff));
          static_cast<float*>(py)[o] = static_cast<float>(fma(0.25, sy, poff));
        }
      }
    }
  }

  __device__ inline void moments(const Raw& r, RT* m) const {
    const CT xs = r.x - cshift;
    const CT ys = r.y - cshift;
    m[0] = xs;
    m[1] = ys;
    if constexpr (NR == 4) {
      const CT d = xs - ys;
      m[2] = xs * ys;
      m[3] = d * d;
    }
  }

  // v += w * (x', y', x'y', (x'-y')^2) of one ring row.  At float64 the four
  // moments pass through LDS in two sub-phases (x', y', then the products),
  // halving the LDS per workgroup; s is the sub-phase (a constant once the
  // engine's sub-phase loop is unrolled) and v holds that sub-phase's two.
  static constexpr int NSUB = sizeof(CT) == 8 ? 2 : 1;
  __device__ inline void vtap(CT w, const RT* m, CT* v, int s) const {
    if constexpr (NSUB == 2) {
      if (s == 0) {
        v[0] = fma(w, m[0], v[0]);
        v[1] = fma(w, m[1], v[1]);
      } else {
        const CT d = m[0] - m[1];
        v[0] = fma(w, m[0] * m[1], v[0]);
        v[1] = fma(w, d * d, v[1]);
      }
    } else {
      v[0] = fma(w, m[0], v[0]);
      v[1] = fma(w, m[1], v[1]);
      v[2] = fma(w, m[2], v[2]);
      v[3] = fma(w, m[3], v[3]);
    }
  }

  // emit reads nothing that the strip engine could load ahead of it (the
  // upstream map of MODE_PREP stays a load in emit: prefetching it would
  // take the float64 kernel past 256 registers, one wave per SIMD)
  struct EIn {};
  __device__ inline EIn emit_load(int, int) const { return EIn{}; }

  // Per output pixel, from the four filtered moments v = (E x', E y', E x'y',
  // E (x'-y')^2) with x' = x - shift, u = E x':
  //   A1 = 2 mu_x mu_y + C1 = 2 ux uy + 2 shift (ux + uy) + (2 shift^2 + C1)
  //   B1 = mu_x^2 + mu_y^2 + C1 = A1 + (ux - uy)^2
  //   A2 = 2 sigma_xy + C2,  sigma_xy = E x'y' - ux uy
  //   B2 = sigma_x^2 + sigma_y^2 + C2 = E (x'-y')^2 + A2 - (ux - uy)^2
  // `valid` masks lanes whose column lies outside the map.
  __device__ inline void emit(int orow, int ocol, const CT* v, bool valid, const EIn&, int) {
    const CT ux = v[0];
    const CT uy = v[1];
    const CT p = ux * uy;
    const CT du = ux - uy;
    const CT A1 = fma(CT(2), p, fma(CT(2) * shift, ux + uy, k1));
    const CT B1 = fma(du, du, A1);
    const CT A2 = fma(CT(2), v[2] - p, C2);
    const CT B2 = fma(-du, du, v[3] + A2);
    if constexpr (MODE == MODE_REDUCE || MODE == MODE_MAP) {
      const CT s = quot(A1 * A2, B1 * B2);
      if constexpr (MODE == MODE_MAP)
        row_store(static_cast<float>(s), row_rsrc(map + out_off + static_cast<int64_t>(orow) * Wout, Wout),
                  lane_off<float>(ocol, valid));
      row_s += valid ? s : CT(0);
    } else if constexpr (MODE == MODE_CS) {
      const CT inv = quot(CT(1), B1 * B2);
      row_s += valid ? A1 * A2 * inv : CT(0);
      row_cs += valid ? A2 * B1 * inv : CT(0);
    } else if constexpr (MODE == MODE_CSF) {
      // the plane sums of MODE_CS, and the MODE_PREP_CS coefficients below
      // with (gS, gCS) = (1 / npix, 0) or (0, 1 / npix)
      const CT inv = CT(1) / (B1 * B2);
      const CT S = A1 * A2 * inv;
      const CT CS = A2 * B1 * inv;
      row_s += valid ? S : CT(0);
      row_cs += valid ? CS : CT(0);
      if (valid) {
        const CT mx = ux + shift;
        const CT my = uy + shift;
        const CT iB1 = B2 * inv;
        const CT iB2 = B1 * inv;
        const CT k = CT(2) * A2 * inv;
        const int64_t idx = out_off + static_cast<int64_t>(orow) * Wout + ocol;
        const CT b = -(gS * S + gCS * CS) * iB2;
        const CT c = CT(2) * (gS * A1 * iB1 + gCS) * iB2;
        const CT dmux = k * (my - mx * A1 * iB1);
        ob[idx] = static_cast<float>(b);
        oc[idx] = static_cast<float>(c);
        otx[idx] = static_cast<float>(gS * dmux - CT(2) * b * ux - c * uy);
        if (oty) {
          const CT dmuy = k * (mx - my * A1 * iB1);
          oty[idx] = static_cast<float>(gS * dmuy - CT(2) * b * uy - c * ux);
        }
      }
    } else if (valid) {
      // the backward coefficients keep their guarded stores: issued on every
      // path (row_store) they measured slower (configs[3] 27.0 -> 32.3 us)
      const CT mx = ux + shift;
      const CT my = uy + shift;
      // one division, 1 / (B1 B2), and each reciprocal from it by a product
      // (B1 >= C1 and B2 >= C2 keep the product far from under- and overflow)
      const CT inv = CT(1) / (B1 * B2);
      const CT iB1 = B2 * inv;
      const CT iB2 = B1 * inv;
      const CT S = A1 * A2 * inv;
      const CT k = CT(2) * A2 * inv;
      const CT dmux = k * (my - mx * A1 * iB1);
      const CT dmuy = k * (mx - my * A1 * iB1);
      const int64_t idx = out_off + static_cast<int64_t>(orow) * Wout + ocol;
      CT b, c, gm;
      if constexpr (MODE == MODE_PREP) {
        gm = dmap ? static_cast<CT>(dmap[idx]) : g_uniform;
        b = -gm * S * iB2;
        c = CT(2) * gm * A1 * iB1 * iB2;
      } else {
        const CT CS = A2 * iB2;
        gm = gS;
        b = -(gS * S + gCS * CS) * iB2;
        c = CT(2) * (gS * A1 * iB1 + gCS) * iB2;
      }
      ob[idx] = static_cast<float>(b);
      oc[idx] = static_cast<float>(c);
      otx[idx] = static_cast<float>(gm * dmux - CT(2) * b * ux - c * uy);
      if (oty) oty[idx] = static_cast<float>(gm * dmuy - CT(2) * b * uy - c * ux);
    }
  }

  // A lane's four outputs of a phase are summed at the compute type, then
  // folded into the float64 lane total.
  __device__ inline void end_row() {
    acc_s += static_cast<double>(row_s);
    acc_cs += static_cast<double>(row_cs);
    row_s = CT(0);
    row_cs = CT(0);
  }
};

// Optional register budget for the float32 forward kernels, in waves per SIMD.
#if defined(FA_SSIM_WPE) && FA_SSIM_WPE > 0
#define FA_SSIM_ATTR __attribute__((amdgpu_waves_per_eu(FA_SSIM_WPE)))
#else
#define FA_SSIM_ATTR
#endif

template <typename T, typename CT, int MODE, int KW, bool LUMA = false>
__global__ __launch_bounds__(BLOCK) FA_SSIM_ATTR void ssim_kernel(SsimArgs a) {
  using Pol = SsimPol<T, CT, MODE, LUMA>;
  __shared__ CT sbuf[2][PH][Pol::NP / Pol::NSUB][HROW];
  __shared__ double sred[2 * WAVES_PER_BLOCK];

  const int t = static_cast<int>(xcd_tile(blockIdx.x, gridDim.x));
  const int plane = t / a.bpp;
  const int tile = t - plane * a.bpp;
  const int chunk = tile / a.strips;
  const int strip = tile - chunk * a.strips;

  Pol pol;
  {
    const int n = plane / a.Cout;
    const int c = plane - n * a.Cout;
#pragma unroll
    for (int ch = 0; ch < Pol::CH; ++ch) {
      const int cc = LUMA ? ch : c;
      pol.x[ch] = static_cast<const T*>(a.x) + n * a.xsn + cc * a.xsc;
      pol.y[ch] = static_cast<const T*>(a.y) + n * a.ysn + cc * a.ysc;
    }
  }
  pol.H = a.H;
  pol.W = a.W;
  pol.shx = static_cast<uint32_t>(a.xsh);
  pol.shy = static_cast<uint32_t>(a.ysh);
  pol.kr = static_cast<CT>(a.kr);
  pol.kg = static_cast<CT>(a.kg);
  pol.kb = static_cast<CT>(a.kb);
  pol.shift = static_cast<CT>(a.shift);
  pol.cshift = static_cast<CT>(a.shift - a.offset);
  pol.poff = a.offset;
  pol.C1 = static_cast<CT>(a.C1);
  pol.C2 = static_cast<CT>(a.C2);
  pol.out_off = static_cast<int64_t>(plane) * a.Hout * a.Wout;
  pol.Wout = a.Wout;
  pol.map = a.map;
  pol.ob = a.ob;
  pol.oc = a.oc;
  pol.otx = a.otx;
  pol.oty = a.oty;
  pol.dmap = a.dmap;
  pol.g_uniform = CT(0);
  pol.gS = CT(0);
  pol.gCS = CT(0);
  if constexpr (MODE == MODE_PREP) {
    if (!a.dmap) pol.g_uniform = static_cast<CT>(a.gscalar[0]) * static_cast<CT>(a.gnorm);
  }
  if constexpr (MODE == MODE_PREP_CS) {
    pol.gS = static_cast<CT>(a.gs[plane]) * static_cast<CT>(a.gnorm);
    pol.gCS = static_cast<CT>(a.gcs[plane]) * static_cast<CT>(a.gnorm);
  }
  if constexpr (MODE == MODE_CSF) {
    pol.gS = a.unit_s ? static_cast<CT>(a.gnorm) : CT(0);
    pol.gCS = a.unit_s ? CT(0) : static_cast<CT>(a.gnorm);
  }
  pol.k1 = static_cast<CT>(2.0 * a.shift * a.shift + a.C1);
  pol.row_s = CT(0);
  pol.row_cs = CT(0);
  pol.acc_s = 0.0;
  pol.acc_cs = 0.0;
  pol.px = a.px;
  pol.py = a.py;
  pol.pool_on = false;
  if constexpr (MODE == MODE_CS || MODE == MODE_CSF) {
    if (a.px) {
      // rows and columns of the output map this workgroup owns, extended to
      // the image edge (2 * floor(H/2), 2 * floor(W/2)) in the last chunk /
      // strip; strip and chunk origins are even, so pairs never straddle
      constexpr int OUTW = StripGeom<KW>::OUTW;
      const int Hd = a.H / 2;
      const int r0 = chunk * a.TH;
      const bool last_chunk = r0 + a.TH >= a.Hout;
      const int c0 = strip * OUTW;
      const bool last_strip = c0 + OUTW >= a.Wout;
      const int col = c0 + static_cast<int>(threadIdx.x);
      const int cend = last_strip ? 2 * (a.W / 2) : c0 + OUTW;
      pol.pool_on = true;
      pol.pool_f64 = a.pool_f64 != 0;
      pol.pool_f16 = a.pool_f16 != 0;
      pol.prow0 = r0;
      pol.prow1 = last_chunk ? 2 * Hd : r0 + a.TH;
      pol.Wd = a.W / 2;
      pol.pool_off = static_cast<int64_t>(plane) * Hd * (a.W / 2);
      pol.pcol_ok = (col & 1) == 0 && col < cend;
      pol.pcol = static_cast<uint32_t>(col >> 1);
    }
  }

  strip_engine<Pol, KW>(pol, a.win, 0, a.Hout, a.Wout, a.TH, strip, chunk, sbuf);

  const int64_t slot = static_cast<int64_t>(plane) * a.bpp + tile;
  if constexpr (MODE == MODE_REDUCE) {
    const double s = block_sum(pol.acc_s, sred);
    if (threadIdx.x == 0) {
      if (a.fin.acc) ssim_fin_add(a.fin, plane / a.Cout, a.Cout * a.bpp, s);
      else a.partial[slot] = s;
    }
  } else if constexpr (MODE == MODE_MAP) {
    const double s = block_sum(pol.acc_s, sred);
    if (threadIdx.x == 0) a.partial[slot] = s;
  } else if constexpr (MODE == MODE_CS || MODE == MODE_CSF) {
    double s = 0.0, scs = 0.0;
    block_sum2(pol.acc_s, pol.acc_cs, sred, &s, &scs);
    if (threadIdx.x == 0) {
      if (a.partial) a.partial[slot] = s;  // null: the cs sums alone were asked for
      a.partial_cs[slot] = scs;
    }
  }
}

// --------------------------------------------------------------------------
// backward scatter: the coefficient maps correlated back onto the full grid
// (zero outside the valid Hout x Wout support) and combined with x', y'.
// --------------------------------------------------------------------------
struct ScatterArgs {
  const void* x;   // float or double, like dx / dy
  const void* y;
  const float* ab;
  const float* ac;
  const float* atx;
  const float* aty;
  void* dx;
  void* dy;
  const float* win;
  int H, W, Hout, Wout, TH, strips, bpp;
  double shift;
  const void* gpx;  // optional gradient of the next pyramid level (2x2 means)
  const void* gpy;
  int gp_f64;       // its element type: float64 (1) or float32 (0)
  const double* gscale;  // optional per-plane factor of the coefficient maps'
                        // share (maps written by MODE_CSF for a unit gradient)
};

template <typename T, bool DY>
struct ScatterPol {
  static constexpr int NP = DY ? 4 : 3;
  using CT = double;
  struct Raw {
    float v[NP];
  };
  // the coefficient maps are float32: the ring keeps them so (half the
  // registers) and each tap widens exactly
  using RT = float;
  static constexpr int NR = NP;

  const float* __restrict__ aux[4];  // this plane of each coefficient map
  int Hout, Wout;
  uint32_t lcol;  // this lane's map column, clamped into the map
  bool col_ok;    // ...and whether it was inside before clamping
  const T* __restrict__ x;
  const T* __restrict__ y;
  int64_t img_off;
  int H, W;
  double shift;
  T* __restrict__ dx;
  T* __restrict__ dy;
  const void* gpx;
  const void* gpy;
  bool gp_f64;
  double gmul;       // this plane's factor of the maps' share (1 without gscale)
  int Hp, Wp;        // pyramid level grid: floor(H/2) x floor(W/2)
  int64_t gp_off;    // this plane of the pyramid gradient

  // Zero padding outside the Hout x Wout support, branch free: the clamped
  // address is always loaded and the value masked.
  __device__ inline void set_column(int col) {
    col_ok = col >= 0 && col < Wout;
    lcol = static_cast<uint32_t>(col < 0 ? 0 : (col < Wout ? col : Wout - 1));
  }

  __device__ inline Raw load(int row) const {
    const bool ok = col_ok && row >= 0 && row < Hout;
    const uint32_t r = static_cast<uint32_t>(row < 0 ? 0 : (row < Hout ? row : Hout - 1));
    const uint32_t o = r * static_cast<uint32_t>(Wout) + lcol;  // uniform row, lane column
    Raw v;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float t = aux[p][o];
      v.v[p] = ok ? t : 0.0f;
    }
    return v;
  }

  __device__ inline void moments(const Raw& r, float* m) const {
#pragma unroll
    for (int p = 0; p < NP; ++p) m[p] = r.v[p];
  }

  // One LDS pass for all maps: splitting the four maps of dy in two halves
  // the LDS per workgroup but takes the kernel to 189 registers, which
  // holds it at two waves per SIMD all the same.
  static constexpr int NSUB = 1;
  __device__ inline void vtap(double w, const float* m, double* v, int) const {
#pragma unroll
    for (int p = 0; p < NP; ++p) v[p] = fma(w, static_cast<double>(m[p]), v[p]);
  }

  __device__ inline void end_row() {}
  __device__ inline void pool2(int, const Raw&, const Raw&) {}

  // A quarter of the pyramid gradient of the 2x2 block this pixel belongs
  // to (the odd trailing row / column belongs to none).
  __device__ inline double pyr_grad(const void* g, int orow, int ocol) const {
    const int pr = orow >> 1, pc = ocol >> 1;
    if (!g || pr >= Hp || pc >= Wp) return 0.0;
    const int64_t o = gp_off + static_cast<int64_t>(pr) * Wp + pc;
    return 0.25 * (gp_f64 ? static_cast<const double*>(g)[o]
                          : static_cast<double>(static_cast<const float*>(g)[o]));
  }

  // Without dy, what emit reads for a lane's COLS_PER_LANE outputs of one
  // row -- x, y and the pyramid gradient of the 2x2 blocks they belong to
  // (the lane's first column is even: outputs k = 0, 1 share block 0, k = 2,
  // 3 block 1) -- is loaded a phase ahead by the strip engine.  With dy the
  // second set of registers would take the kernel past 256 (one wave per
  // SIMD), so emit loads it itself.
  static constexpr bool PRE = !DY;
  struct EInPre {
    T x[COLS_PER_LANE], y[COLS_PER_LANE];
    double g[2];
  };
  struct EInNone {};
  using EIn = typename std::conditional<PRE, EInPre, EInNone>::type;

  __device__ inline EIn emit_load(int orow, int ocol) const {
    EIn e;
    if constexpr (PRE) {
      const int r = orow < H ? orow : H - 1;
      const int64_t base = img_off + static_cast<int64_t>(r) * W;
#pragma unroll
      for (int k = 0; k < COLS_PER_LANE; ++k) {
        const int c = ocol + k < W ? ocol + k : W - 1;
        e.x[k] = x[base + c];
        e.y[k] = y[base + c];
      }
      e.g[0] = 0.0;
      e.g[1] = 0.0;
      if (gpx && Hp > 0 && Wp > 0) {  // uniform
        const int pr = orow >> 1;
        const int64_t prow = gp_off + static_cast<int64_t>(pr < Hp ? pr : Hp - 1) * Wp;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int pc = (ocol >> 1) + j;
          const int64_t o = prow + (pc < Wp ? pc : Wp - 1);
          const double t = gp_f64 ? static_cast<const double*>(gpx)[o]
                                  : static_cast<double>(static_cast<const float*>(gpx)[o]);
          e.g[j] = pr < Hp && pc < Wp ? 0.25 * t : 0.0;
        }
      }
    }
    return e;
  }

  __device__ inline void emit(int orow, int ocol, const double* v, bool valid, const EIn& e,
                              int k) {
    if constexpr (PRE) {
      // every lane stores, through a row buffer resource (see row_store)
      const double xv = static_cast<double>(e.x[k]) - shift;
      const double yv = static_cast<double>(e.y[k]) - shift;
      row_store(static_cast<T>(gmul * (2.0 * xv * v[0] + yv * v[1] + v[2]) + e.g[k >> 1]),
                row_rsrc(dx ? dx + img_off + static_cast<int64_t>(orow) * W : nullptr, W),
                lane_off<T>(ocol, valid));
    } else {
      if (!valid) return;
      const int64_t o = img_off + static_cast<int64_t>(orow) * W + ocol;
      const double xv = static_cast<double>(x[o]) - shift;
      const double yv = static_cast<double>(y[o]) - shift;
      if (dx)
        dx[o] = static_cast<T>(gmul * (2.0 * xv * v[0] + yv * v[1] + v[2]) +
                               pyr_grad(gpx, orow, ocol));
      dy[o] = static_cast<T>(gmul * (2.0 * yv * v[0] + xv * v[1] + v[3]) +
                             pyr_grad(gpy, orow, ocol));
    }
  }
};

template <typename T, int KW, bool DY>
__global__ __launch_bounds__(BLOCK) void scatter_kernel(ScatterArgs a) {
  constexpr int NP = ScatterPol<T, DY>::NP;
  __shared__ double sbuf[2][PH][NP / ScatterPol<T, DY>::NSUB][HROW];

  const int t = static_cast<int>(xcd_tile(blockIdx.x, gridDim.x));
  const int plane = t / a.bpp;
  const int tile = t - plane * a.bpp;
  const int chunk = tile / a.strips;
  const int strip = tile - chunk * a.strips;

  ScatterPol<T, DY> pol;
  const int64_t aux_off = static_cast<int64_t>(plane) * a.Hout * a.Wout;
  pol.aux[0] = a.ab + aux_off;
  pol.aux[1] = a.ac + aux_off;
  pol.aux[2] = a.atx + aux_off;
  pol.aux[3] = DY ? a.aty + aux_off : nullptr;
  pol.Hout = a.Hout;
  pol.Wout = a.Wout;
  pol.x = static_cast<const T*>(a.x);
  pol.y = static_cast<const T*>(a.y);
  pol.img_off = static_cast<int64_t>(plane) * a.H * a.W;
  pol.H = a.H;
  pol.W = a.W;
  pol.shift = a.shift;
  pol.dx = static_cast<T*>(a.dx);
  pol.dy = static_cast<T*>(a.dy);
  pol.gpx = a.gpx;
  pol.gpy = a.gpy;
  pol.gp_f64 = a.gp_f64 != 0;
  // x * 1.0 is x: without gscale the results are those of the plain scatter
  pol.gmul = a.gscale ? a.gscale[plane] : 1.0;
  pol.Hp = a.H / 2;
  pol.Wp = a.W / 2;
  pol.gp_off = static_cast<int64_t>(plane) * pol.Hp * pol.Wp;
  strip_engine<ScatterPol<T, DY>, KW>(pol, a.win, -(KW - 1), a.H, a.W, a.TH, strip, chunk,
                                      sbuf);
}

// Per-plane means of two partial arrays (MS-SSIM keeps planes apart).
__global__ __launch_bounds__(BLOCK) void planes2_kernel(const double* __restrict__ pa,
                                                        const double* __restrict__ pb,
                                                        int ncols, double npix,
                                                        double* __restrict__ oa,
                                                        double* __restrict__ ob) {
  __shared__ double smem[2 * WAVES_PER_BLOCK];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * ncols;
  double a = 0.0, b = 0.0;
  for (int i = threadIdx.x; i < ncols; i += BLOCK) {
    a += pa[base + i];
    b += pb[base + i];
  }
  double sa = 0.0, sb = 0.0;
  block_sum2(a, b, smem, &sa, &sb);
  if (threadIdx.x == 0) {
    oa[blockIdx.x] = sa / npix;
    ob[blockIdx.x] = sb / npix;
  }
}

// MS-SSIM's last steps (reference functional.py:897-901) straight from the
// per-scale partial sums the CS passes left.  One workgroup per (plane,
// scale) reduces that scale's slots in the order planes2_kernel uses (so the
// plane terms are the same bits), clamps at zero and raises to the scale's
// weight; one more workgroup multiplies over the scales and takes the channel
// mean of each image and the mean over the batch.
constexpr int MS_MAX_SCALES = 8;
struct MsParts {
  const double* p[MS_MAX_SCALES];  // per scale: planes * slots[m] partial sums
  int slots[MS_MAX_SCALES];
  double npix[MS_MAX_SCALES];      // output pixels of one plane at that scale
  double w[MS_MAX_SCALES];
};

// grid (planes, M): terms[m * planes + plane] = max(plane mean, 0)^w[m] at scale m
__global__ __launch_bounds__(BLOCK) void ms_term_kernel(MsParts parts,
                                                        double* __restrict__ terms) {
  __shared__ double smem[WAVES_PER_BLOCK];
  const int plane = blockIdx.x;
  const int m = blockIdx.y;
  const int n = parts.slots[m];
  const double* src = parts.p[m] + static_cast<int64_t>(plane) * n;
  double a = 0.0;
  for (int i = threadIdx.x; i < n; i += BLOCK) a += src[i];
  const double sum = block_sum(a, smem);
  if (threadIdx.x == 0) {
    const double v = sum / parts.npix[m];
    // clamp at zero like torch's clamp_min: a NaN term stays NaN (so does the
    // product), it is not clamped to a finite 0
    const double c = (v != v) ? v : (v > 0.0 ? v : 0.0);
    terms[static_cast<int64_t>(m) * gridDim.x + plane] = pow(c, parts.w[m]);
  }
}

__global__ __launch_bounds__(BLOCK) void ms_finish_kernel(int M, int N, int C,
                                                          double* __restrict__ terms,
                                                          double* __restrict__ out_per_image,
                                                          double* __restrict__ out_total) {
  __shared__ double smem[WAVES_PER_BLOCK];
  const int64_t planes = static_cast<int64_t>(N) * C;
  // each thread turns its planes' terms into the product over the scales,
  // kept in the scale-0 row of `terms`
  for (int64_t p = threadIdx.x; p < planes; p += BLOCK) {
    double prod = 1.0;
    for (int m = 0; m < M; ++m) prod *= terms[m * planes + p];
    terms[p] = prod;
  }
  __syncthreads();  // global writes of this workgroup are visible to it after the barrier
  double tot = 0.0;
  for (int n = threadIdx.x; n < N; n += BLOCK) {
    double img = 0.0;
    for (int c = 0; c < C; ++c) img += terms[static_cast<int64_t>(n) * C + c];
    img /= static_cast<double>(C);
    if (out_per_image) out_per_image[n] = img;
    tot += img;
  }
  tot = block_sum(tot, smem);
  if (threadIdx.x == 0 && out_total) *out_total = tot / static_cast<double>(N);
}

// MS-SSIM's head over plane means that are already formed (the training
// path, where each scale's means are outputs of its own pass): per plane the
// product over the scales of max(t_m, 0)^w_m, the mean over the C channels of
// each image and the batch mean (fa_gpu_ms_ssim_head), and the gradient of
// every scale's plane means from the upstream gradient of either mean
// (fa_gpu_ms_ssim_head_backward).  The clamp and the power differentiate as
// torch's clamp_min and pow do (reference functional.py:897-901 combines the
// scales with them): no gradient where t < 0 (or t is NaN) or w = 0, and
// w * 0^(w - 1) = inf for a zero factor under a fractional weight.
struct MsHead {
  const double* t[MS_MAX_SCALES];  // scale m's plane means, N * C each
  double w[MS_MAX_SCALES];
  int M, N, C;
};

struct MsHeadGrads {
  double* g[MS_MAX_SCALES];  // scale m's gradient, N * C (null: not wanted)
};

__device__ inline double ms_clamp0(double v) { return (v != v) ? v : (v > 0.0 ? v : 0.0); }

// The forward's factors wait in LDS, MS_HEAD_LDS doubles: whole images of
// planes at a time (every thread one factor, every factor's power computed
// at once instead of in one thread's chain).
constexpr int MS_HEAD_LDS = BLOCK * MS_MAX_SCALES;

// One workgroup.  A chunk of images: each thread raises one (scale, plane)
// mean to its weight, then each plane's product, then each image's channel
// mean; thread i keeps images i, i + BLOCK, ... of every chunk for the batch
// sum, so the sum's order does not depend on timing.  Images whose C * M
// factors exceed the LDS take the slow path (one thread per image).
__global__ __launch_bounds__(BLOCK) void ms_head_kernel(MsHead h,
                                                        double* __restrict__ out_per_image,
                                                        double* __restrict__ out_total) {
  __shared__ double sf[MS_HEAD_LDS];
  __shared__ double smem[WAVES_PER_BLOCK];
  const int64_t per_img = static_cast<int64_t>(h.C) * h.M;  // factors of one image
  const int ci = per_img <= MS_HEAD_LDS ? static_cast<int>(MS_HEAD_LDS / per_img) : 0;  // images per chunk
  double tot = 0.0;
  if (ci == 0) {
    for (int n = threadIdx.x; n < h.N; n += BLOCK) {
      double img = 0.0;
      for (int c = 0; c < h.C; ++c) {
        const int64_t p = static_cast<int64_t>(n) * h.C + c;
        double prod = 1.0;
        for (int m = 0; m < h.M; ++m) prod *= pow(ms_clamp0(h.t[m][p]), h.w[m]);
        img += prod;
      }
      img /= static_cast<double>(h.C);
      if (out_per_image) out_per_image[n] = img;
      tot += img;
    }
  } else {
    for (int n0 = 0; n0 < h.N; n0 += ci) {
      const int nimg = min(ci, h.N - n0);
      const int cp = nimg * h.C;  // planes of the chunk
      const int64_t p0 = static_cast<int64_t>(n0) * h.C;
      for (int i = threadIdx.x; i < cp * h.M; i += BLOCK) {
        const int m = i / cp;
        sf[i] = pow(ms_clamp0(h.t[m][p0 + (i - m * cp)]), h.w[m]);
      }
      __syncthreads();
      for (int q = threadIdx.x; q < cp; q += BLOCK) {  // column q is this thread's alone
        double prod = sf[q];
        for (int m = 1; m < h.M; ++m) prod *= sf[m * cp + q];
        sf[q] = prod;
      }
      __syncthreads();
      for (int i = threadIdx.x; i < nimg; i += BLOCK) {
        double img = 0.0;
        for (int c = 0; c < h.C; ++c) img += sf[i * h.C + c];
        img /= static_cast<double>(h.C);
        if (out_per_image) out_per_image[n0 + i] = img;
        tot += img;
      }
      __syncthreads();  // the next chunk overwrites sf
    }
  }
  tot = block_sum(tot, smem);
  if (threadIdx.x == 0 && out_total) *out_total = tot / static_cast<double>(h.N);
}

// BLOCK / MS_MAX_SCALES planes per workgroup, thread (q, m) = (tid / 8,
// tid % 8): the factor and the power's derivative of scale m's mean of plane
// q; the factors meet in LDS for each thread's product of the others.
// g_per_image (N) or g_total (1): the upstream gradient of the per-image
// values or of the batch mean.
constexpr int MS_HEAD_BW_PLANES = BLOCK / MS_MAX_SCALES;

__global__ __launch_bounds__(BLOCK) void ms_head_backward_kernel(
    MsHead h, const double* __restrict__ g_per_image, const double* __restrict__ g_total,
    MsHeadGrads out) {
  __shared__ double sf[MS_HEAD_BW_PLANES][MS_MAX_SCALES];
  const int planes = h.N * h.C;  // <= INT32_MAX - BLOCK (host check)
  const int q = static_cast<int>(threadIdx.x) / MS_MAX_SCALES;
  const int m = static_cast<int>(threadIdx.x) % MS_MAX_SCALES;
  const int p = static_cast<int>(blockIdx.x) * MS_HEAD_BW_PLANES + q;
  const bool live = p < planes && m < h.M;
  double t = 1.0, f = 1.0;
  if (live) {
    t = h.t[m][p];
    f = pow(ms_clamp0(t), h.w[m]);
  }
  sf[q][m] = f;  // 1.0 for the scales past M
  __syncthreads();
  if (!live || !out.g[m]) return;
  const int n = p / h.C;
  // the means' backward: 1 / N, then 1 / C, as torch's mean backward divides
  const double gi = g_per_image ? g_per_image[n] : g_total[0] / static_cast<double>(h.N);
  const double gp = gi / static_cast<double>(h.C);
  double others = 1.0;  // the product of the other factors, exact where some are zero
#pragma unroll
  for (int k = 0; k < MS_MAX_SCALES; ++k)
    if (k != m) others *= sf[q][k];
  const double dpow = h.w[m] == 0.0 ? 0.0 : h.w[m] * pow(ms_clamp0(t), h.w[m] - 1.0);
  out.g[m][p] = t >= 0.0 ? (gp * others) * dpow : 0.0;
}

// --------------------------------------------------------------------------
// host dispatch
// --------------------------------------------------------------------------
// Workgroups of this kernel one CU holds at once.
static int occupancy_wgs(const void* fn) {
  int v = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, fn, BLOCK, 0) != hipSuccess || v <= 0)
    v = 1;
  return v;
}

// Workgroups of a strip-engine launch over `planes` planes; the grid is 1-D.
static int grid_of(int64_t planes, int64_t per_plane, dim3* grid) {
  const int64_t total = planes * per_plane;
  if (total <= 0 || total > (static_cast<int64_t>(INT32_MAX) / BLOCK)) return FA_E_SHAPE;
  *grid = dim3(static_cast<unsigned>(total));
  return FA_OK;
}

// The plan of a launch, checked once its tiles are known: other launches
// need nothing more; an SSIM forward that asked for the one-launch finish
// needs its counts to fit (Cout * tiles contributions per image word), and
// without the finish, the partial slots (false: refused, nothing launched).
template <typename Args>
static bool strip_plan_ok(Args&) {
  return true;
}
static bool strip_plan_ok(SsimArgs& a) {
  if (!a.fin.acc) return true;
  if (static_cast<int64_t>(a.Cout) * a.bpp < (int64_t(1) << SSIM_FIN_COUNT_BITS)) return true;
  a.fin.acc = nullptr;
  return a.partial != nullptr;
}

// Tiles `kern` over `planes` planes of an out_H x out_W grid for its
// occupancy `occ` and launches it; a.TH / a.strips / a.bpp report the tiling.
template <typename Args>
static int launch_strips(void (*kern)(Args), int occ, Args& a, int64_t planes, int out_H,
                         int out_W, int K, int device, hipStream_t st) {
  const Tiling t = tiling_for(planes, out_H, out_W, K, static_cast<int64_t>(cu_count(device)) * occ);
  a.TH = t.TH;
  a.strips = t.strips;
  a.bpp = t.tiles;
  if (!strip_plan_ok(a)) return FA_E_ARG;  // nothing launched
  dim3 grid;
  const int rc = grid_of(planes, t.tiles, &grid);
  if (rc != FA_OK) return rc;
  hipLaunchKernelGGL(kern, grid, dim3(BLOCK), 0, st, a);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

template <typename T, typename CT, int MODE, int KW, bool LUMA>
static int launch_ssim_kw(SsimArgs& a, int64_t planes, int device, hipStream_t st) {
  static const int occ =
      occupancy_wgs(reinterpret_cast<const void*>(&ssim_kernel<T, CT, MODE, KW, LUMA>));
  return launch_strips(ssim_kernel<T, CT, MODE, KW, LUMA>, occ, a, planes, a.Hout, a.Wout,
                       KW, device, st);
}

template <typename T, typename CT, int MODE, bool LUMA = false>
static int launch_ssim_k(int K, SsimArgs& a, int64_t planes, int device, hipStream_t st) {
  switch (K) {
    case 3: return launch_ssim_kw<T, CT, MODE, 3, LUMA>(a, planes, device, st);
    case 5: return launch_ssim_kw<T, CT, MODE, 5, LUMA>(a, planes, device, st);
    case 7: return launch_ssim_kw<T, CT, MODE, 7, LUMA>(a, planes, device, st);
    case 9: return launch_ssim_kw<T, CT, MODE, 9, LUMA>(a, planes, device, st);
    case 11: return launch_ssim_kw<T, CT, MODE, 11, LUMA>(a, planes, device, st);
    default: return FA_E_WINDOW;
  }
}

template <int MODE, bool LUMA>
static int launch_ssim_t(int dtype, int K, SsimArgs& a, int64_t planes, int device,
                         hipStream_t st) {
  switch (dtype) {
    case FA_U8: return launch_ssim_k<uint8_t, float, MODE, LUMA>(K, a, planes, device, st);
    case FA_F16: return launch_ssim_k<half_t, float, MODE, LUMA>(K, a, planes, device, st);
    case FA_BF16: return launch_ssim_k<bf16_t, float, MODE, LUMA>(K, a, planes, device, st);
    case FA_F32: return launch_ssim_k<float, float, MODE, LUMA>(K, a, planes, device, st);
    case FA_F64: return launch_ssim_k<double, double, MODE, LUMA>(K, a, planes, device, st);
    default: return FA_E_DTYPE;
  }
}

// Forward launches: with luma (a.Cout == 1 over three input channels) or not.
template <int MODE>
static int launch_ssim(int dtype, int K, bool luma, SsimArgs& a, int64_t planes, int device,
                       hipStream_t st) {
  return luma ? launch_ssim_t<MODE, true>(dtype, K, a, planes, device, st)
              : launch_ssim_t<MODE, false>(dtype, K, a, planes, device, st);
}

template <typename T, int KW, bool DY>
static int launch_scatter_kw(ScatterArgs& a, int64_t planes, int device, hipStream_t st) {
  static const int occ = occupancy_wgs(reinterpret_cast<const void*>(&scatter_kernel<T, KW, DY>));
  return launch_strips(scatter_kernel<T, KW, DY>, occ, a, planes, a.H, a.W, KW, device, st);
}

template <typename T, bool DY>
static int launch_scatter_k(int K, ScatterArgs& a, int64_t planes, int device,
                            hipStream_t st) {
  switch (K) {
    case 3: return launch_scatter_kw<T, 3, DY>(a, planes, device, st);
    case 5: return launch_scatter_kw<T, 5, DY>(a, planes, device, st);
    case 7: return launch_scatter_kw<T, 7, DY>(a, planes, device, st);
    case 9: return launch_scatter_kw<T, 9, DY>(a, planes, device, st);
    case 11: return launch_scatter_kw<T, 11, DY>(a, planes, device, st);
    default: return FA_E_WINDOW;
  }
}

// Validates the common SSIM arguments and derives the output geometry.
static int ssim_shape(int N, int C, int H, int W, int K, int* Hout, int* Wout) {
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return FA_E_SHAPE;
  if (static_cast<int64_t>(H) * W > INT32_MAX) return FA_E_SHAPE;  // 32-bit plane offsets
  if (K < 3 || K > FA_MAX_WIN || (K & 1) == 0) return FA_E_WINDOW;
  *Hout = H - K + 1;
  *Wout = W - K + 1;
  if (*Hout <= 0 || *Wout <= 0) return FA_E_SHAPE;
  return FA_OK;
}

// Fills the input views of `a` (null strides: contiguous N x C x H x W) and
// the luma transform {kr, kg, kb, offset} (null: none; otherwise C must be 3
// and each image is one plane).  Row offsets within a plane stay 32-bit.
static int set_views(SsimArgs& a, int C, int H, int W, const int64_t* xs, const int64_t* ys,
                     const double* luma) {
  const int64_t plane = static_cast<int64_t>(H) * W;
  const int64_t vx[3] = {xs ? xs[0] : plane * C, xs ? xs[1] : plane, xs ? xs[2] : W};
  const int64_t vy[3] = {ys ? ys[0] : plane * C, ys ? ys[1] : plane, ys ? ys[2] : W};
  for (int i = 0; i < 3; ++i)
    if (vx[i] < 0 || vy[i] < 0) return FA_E_SHAPE;
  // rows may not overlap, and a plane's last element must be 32-bit addressable
  if (vx[2] < W || vy[2] < W) return FA_E_SHAPE;
  if ((H - 1) * vx[2] + W > INT32_MAX || (H - 1) * vy[2] + W > INT32_MAX) return FA_E_SHAPE;
  if (luma && C != 3) return FA_E_SHAPE;
  a.xsn = vx[0];
  a.xsc = vx[1];
  a.xsh = static_cast<int>(vx[2]);
  a.ysn = vy[0];
  a.ysc = vy[1];
  a.ysh = static_cast<int>(vy[2]);
  a.Cout = luma ? 1 : C;
  if (luma) {
    a.kr = luma[0];
    a.kg = luma[1];
    a.kb = luma[2];
    a.offset = luma[3];
  }
  return FA_OK;
}

// The scatter of coefficient maps `aux` (b, c, tx and, with aux_dy, ty, each
// N * C * Hout * Wout float32) onto dx / dy, optionally scaled per plane by
// gscale, plus a quarter of the pyramid level's gradient over each 2x2 block.
template <typename T>
static int scatter_impl(const T* x, const T* y, const double* gscale, const float* win, int K,
                        int N, int C, int H, int W, double shift, const float* aux, bool aux_dy,
                        const void* gpx, const void* gpy, int gp_dtype, T* dx, T* dy,
                        int device, hipStream_t st) {
  int Hout = 0, Wout = 0;
  const int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  if (dy && !aux_dy) return FA_E_ARG;
  const int64_t planes = static_cast<int64_t>(N) * C;
  const int64_t aux_stride = planes * Hout * Wout;
  ScatterArgs s = {};
  s.x = x;
  s.y = y;
  s.ab = aux;
  s.ac = aux + aux_stride;
  s.atx = aux + 2 * aux_stride;
  s.aty = aux_dy ? aux + 3 * aux_stride : nullptr;
  s.dx = dx;
  s.dy = dy;
  s.win = win;
  s.H = H;
  s.W = W;
  s.Hout = Hout;
  s.Wout = Wout;
  s.shift = shift;
  s.gpx = gpx;
  s.gpy = gpy;
  s.gp_f64 = gp_dtype == FA_F64 ? 1 : 0;
  s.gscale = gscale;
  return dy ? launch_scatter_k<T, true>(K, s, planes, device, st)
            : launch_scatter_k<T, false>(K, s, planes, device, st);
}

// The coefficient pass plus the scatter, shared by the backward entry points.
// T is the element type of x, y, dx and dy (float, or double for the float64
// MS-SSIM pyramid levels); the arithmetic is float64 either way.
template <typename T, int MODE>
static int ssim_backward_impl(const T* x, const T* y, const float* dmap,
                              const float* gscalar, const float* gs,
                              const float* gcs, const float* win, int K, int N,
                              int C, int H, int W, double shift, double C1,
                              double C2, float* aux, T* dx, T* dy,
                              const void* gpx, const void* gpy, int gp_dtype,
                              int device, hipStream_t st) {
  int Hout = 0, Wout = 0;
  int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  const int64_t planes = static_cast<int64_t>(N) * C;
  const int64_t npix = static_cast<int64_t>(Hout) * Wout;
  const int64_t aux_stride = planes * npix;

  SsimArgs a = {};
  a.x = x;
  a.y = y;
  a.H = H;
  a.W = W;
  a.Hout = Hout;
  a.Wout = Wout;
  rc = set_views(a, C, H, W, nullptr, nullptr, nullptr);
  if (rc != FA_OK) return rc;
  a.shift = shift;
  a.C1 = C1;
  a.C2 = C2;
  a.win = win;
  a.dmap = dmap;
  a.gscalar = gscalar;
  a.gs = gs;
  a.gcs = gcs;
  a.gnorm = MODE == MODE_PREP ? 1.0 / (static_cast<double>(npix) * static_cast<double>(planes))
                              : 1.0 / static_cast<double>(npix);
  a.ob = aux;
  a.oc = aux + aux_stride;
  a.otx = aux + 2 * aux_stride;
  a.oty = dy ? aux + 3 * aux_stride : nullptr;
  rc = launch_ssim_k<T, double, MODE>(K, a, planes, device, st);
  if (rc != FA_OK) return rc;
  return scatter_impl<T>(x, y, nullptr, win, K, N, C, H, W, shift, aux, dy != nullptr, gpx, gpy,
                         gp_dtype, dx, dy, device, st);
}

// fa_gpu_ssim_cs over views, with optional luma and, when px / py are not
// null, the next pyramid level.
static int ssim_cs_impl(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                        const int64_t* xs, const int64_t* ys, const double* luma,
                        const float* win, int K, double shift, double C1, double C2,
                        double* partial, double* partial_cs, int bpp, double* out_s,
                        double* out_cs, int* out_slots, void* px, void* py, int pool_dtype,
                        int device, void* stream) {
  if (!x || !y || !win || !partial_cs) return FA_E_ARG;
  // partial may be null only when nothing is finalized: then the pass forms
  // the cs sums alone (all MS-SSIM reads below its coarsest scale)
  if (!partial && (out_s || out_cs)) return FA_E_ARG;
  // FA_DTYPE_U8_PYRAMID: float32 samples of a uint8 pyramid level, or
  // float16 samples of its first level (a hint that admits the matrix-core
  // kernel; the strip kernel reads plain float32 / float16)
  const bool u8_pyramid = (dtype & FA_DTYPE_U8_PYRAMID) != 0;
  dtype &= ~FA_DTYPE_U8_PYRAMID;
  if (u8_pyramid && dtype != FA_F32 && dtype != FA_F16) return FA_E_DTYPE;
  // plane means, or (both null) the partial sums left for fa_gpu_ms_ssim_reduce
  if ((out_s == nullptr) != (out_cs == nullptr)) return FA_E_ARG;
  if (!out_s && !out_slots) return FA_E_ARG;
  if ((px == nullptr) != (py == nullptr)) return FA_E_ARG;
  int Hout = 0, Wout = 0;
  int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  if (bpp != ssim_slots(Hout, Wout, K)) return FA_E_ARG;
  SsimArgs a = {};
  rc = set_views(a, C, H, W, xs, ys, luma);
  if (rc != FA_OK) return rc;
  const int64_t planes = static_cast<int64_t>(N) * a.Cout;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);

  a.x = x;
  a.y = y;
  a.H = H;
  a.W = W;
  a.Hout = Hout;
  a.Wout = Wout;
  a.shift = shift;
  a.C1 = C1;
  a.C2 = C2;
  a.win = win;
  a.partial = partial;
  a.partial_cs = partial_cs;
  a.px = px;
  a.py = py;
  a.pool_f64 = pool_dtype == FA_F64 ? 1 : 0;
  a.pool_f16 = pool_dtype == FA_F16 ? 1 : 0;
  int tiles = 0;
  if ((dtype == FA_U8 || u8_pyramid) && !luma &&
      (!px || pool_dtype == FA_F32 || pool_dtype == FA_F16)) {
    // uint8 planes and the levels of their pyramid: the matrix-core kernel
    // when the layout allows (fa_ssim_mfma.hip), next level included
    const int src = !u8_pyramid        ? SsimMfmaCall::U8
                    : dtype == FA_F16 ? SsimMfmaCall::F16_LEVEL
                                      : SsimMfmaCall::F32_LEVEL;
    const SsimMfmaCall mc = {x, y, src, a.xsn, a.xsc, a.ysn, a.ysc, a.xsh, a.ysh,
                             N, C, H, W, Hout, Wout, K, win, C1, C2, nullptr, partial, bpp,
                             partial_cs, px, py, px != nullptr && pool_dtype == FA_F16};
    rc = ssim_mfma(mc, device, st, &tiles);
    if (rc != FA_OK) return rc;
  }
  if (tiles == 0) {
    rc = launch_ssim<MODE_CS>(dtype, K, luma != nullptr, a, planes, device, st);
    if (rc != FA_OK) return rc;
    tiles = a.bpp;
  }
  if (out_slots) *out_slots = tiles;  // the launch packed each plane's partials this densely
  if (!out_s) return FA_OK;
  hipLaunchKernelGGL(planes2_kernel, dim3(static_cast<unsigned>(planes)), dim3(BLOCK), 0, st,
                     partial, partial_cs, tiles, static_cast<double>(Hout) * Wout, out_s,
                     out_cs);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// fa_gpu_ssim over views, with optional luma.
static int ssim_impl(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                     const int64_t* xs, const int64_t* ys, const double* luma,
                     const float* win, int K, double shift, double C1, double C2,
                     float* map_out, double* partial, int bpp, double* out_per_image,
                     double* out_total, int device, void* stream, uint64_t* acc = nullptr) {
  // a null workspace is enough only where the matrix-core launch finishes the
  // call (ssim_mfma refuses it otherwise, before launching)
  if (!x || !y || !win || (!partial && !acc)) return FA_E_ARG;
  int Hout = 0, Wout = 0;
  int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  if (bpp != ssim_slots(Hout, Wout, K)) return FA_E_ARG;
  SsimArgs a = {};
  rc = set_views(a, C, H, W, xs, ys, luma);
  if (rc != FA_OK) return rc;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);

  a.x = x;
  a.y = y;
  a.H = H;
  a.W = W;
  a.Hout = Hout;
  a.Wout = Wout;
  a.shift = shift;
  a.C1 = C1;
  a.C2 = C2;
  a.win = win;
  a.map = map_out;
  a.partial = partial;
  const int Cout = a.Cout;
  const int64_t planes = static_cast<int64_t>(N) * Cout;
  const bool lm = luma != nullptr;
  int tiles = 0;
  if (dtype == FA_U8 && !lm) {
    // uint8 planes: both Gaussian passes on the matrix cores when the layout
    // allows (fa_ssim_mfma.hip); otherwise the strip kernel below
    const SsimMfmaCall mc = {x, y, SsimMfmaCall::U8, a.xsn, a.xsc, a.ysn, a.ysc, a.xsh, a.ysh,
                             N, C, H, W, Hout, Wout, K, win, C1, C2, map_out, partial, bpp,
                             nullptr, nullptr, nullptr, false, acc, out_per_image, out_total};
    rc = ssim_mfma(mc, device, st, &tiles);
    if (rc != FA_OK) return rc;
    if (tiles < 0) return FA_OK;  // the launch finished the call
  }
  if (tiles == 0) {
    // the strip kernel's own one-launch finish: the mean alone, as the
    // matrix-core kernel's (at most SSIM_FIN_MAX_IMAGES images, C1, C2 > 0 so
    // that no SSIM value is NaN); launch_strips drops it where the counts do
    // not fit, and then needs the workspace
    if (acc && !map_out && N <= SSIM_FIN_MAX_IMAGES && (out_per_image || out_total) &&
        C1 > 0.0 && C2 > 0.0) {
      a.fin.acc = acc;
      a.fin.N = N;
      a.fin.npix_img = static_cast<double>(Hout) * Wout * Cout;
      a.fin.npix_all = a.fin.npix_img * N;
      a.fin.out_per_image = out_per_image;
      a.fin.out_total = out_total;
      if (!ssim_fin_scale(a.fin)) a.fin.acc = nullptr;
    }
    if (!partial && !a.fin.acc) return FA_E_ARG;  // nothing launched
    rc = map_out ? launch_ssim<MODE_MAP>(dtype, K, lm, a, planes, device, st)
                 : launch_ssim<MODE_REDUCE>(dtype, K, lm, a, planes, device, st);
    if (rc != FA_OK) return rc;
    if (a.fin.acc) return FA_OK;  // the launch finished the call
    tiles = a.bpp;
  } else if (!partial) {
    return FA_E_ARG;
  }

  // each image owns Cout * tiles consecutive slots of `partial`
  const double npix = static_cast<double>(Hout) * Wout;
  return launch_finalize(partial, false, N, Cout * tiles, npix * Cout,
                         npix * Cout * static_cast<double>(N), FA_PSNR_NONE,
                         out_per_image, out_total, nullptr, nullptr, st);
}

// MS-SSIM's reduction (fa_gpu_ms_ssim_reduce, and the end of fa_gpu_ms_ssim).
static int ms_reduce_impl(const double* const* partials, const int* slots, const double* npix,
                          const double* weights, int M, int N, int C, double* plane_scratch,
                          double* out_per_image, double* out_total, int device, void* stream) {
  if (!partials || !slots || !npix || !weights || !plane_scratch) return FA_E_ARG;
  if (M <= 0 || M > MS_MAX_SCALES || N <= 0 || C <= 0) return FA_E_SHAPE;
  if (!out_per_image && !out_total) return FA_E_ARG;
  const int64_t planes = static_cast<int64_t>(N) * C;
  if (planes > INT32_MAX) return FA_E_SHAPE;
  MsParts parts = {};
  for (int m = 0; m < M; ++m) {
    if (!partials[m]) return FA_E_ARG;
    if (slots[m] <= 0 || !(npix[m] > 0.0)) return FA_E_SHAPE;
    parts.p[m] = partials[m];
    parts.slots[m] = slots[m];
    parts.npix[m] = npix[m];
    parts.w[m] = weights[m];
  }
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ms_term_kernel, dim3(static_cast<unsigned>(planes), M), dim3(BLOCK), 0, st,
                     parts, plane_scratch);
  FA_LAUNCH_CHECK();
  hipLaunchKernelGGL(ms_finish_kernel, dim3(1), dim3(BLOCK), 0, st, M, N, C, plane_scratch,
                     out_per_image, out_total);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// The layout of fa_gpu_ms_ssim's workspace and the per-scale shapes and
// element types: the exact pyramid of the inference path (float16 first level
// and float32 below it under uint8 input, float64 under floating input or a
// luma plane), each scale's partial sums (the cs sums, and the SSIM sums at
// the coarsest scale) and the reduction's scratch, every piece 256-byte
// aligned.  Every scale's shape is checked here, before anything runs.
struct MsPlan {
  int M, cout;
  int H[MS_MAX_SCALES], W[MS_MAX_SCALES], bpp[MS_MAX_SCALES];
  int in_dtype[MS_MAX_SCALES];     // dtype code of scale i's input
  int level_dtype[MS_MAX_SCALES];  // element type of level i (i >= 1)
  int64_t level_x[MS_MAX_SCALES], level_y[MS_MAX_SCALES];  // byte offsets (i >= 1)
  int64_t pcs[MS_MAX_SCALES], ps_last, scratch, total;
};

static int ms_plan(int dtype, int N, int C, int H, int W, int K, int M, bool luma, MsPlan* p) {
  if (dtype < FA_U8 || dtype > FA_F64) return FA_E_DTYPE;
  if (M <= 0 || M > MS_MAX_SCALES || N <= 0 || C <= 0) return FA_E_SHAPE;
  if (luma && C != 3) return FA_E_SHAPE;
  p->M = M;
  p->cout = luma ? 1 : C;
  const int64_t planes = static_cast<int64_t>(N) * p->cout;
  const bool u8 = dtype == FA_U8 && !luma;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  for (int i = 0; i < M; ++i) {
    p->H[i] = i == 0 ? H : p->H[i - 1] / 2;
    p->W[i] = i == 0 ? W : p->W[i - 1] / 2;
    int Hout = 0, Wout = 0;
    const int rc = ssim_shape(N, i == 0 ? C : p->cout, p->H[i], p->W[i], K, &Hout, &Wout);
    if (rc != FA_OK) return rc;
    p->bpp[i] = ssim_slots(Hout, Wout, K);
    if (i > 0) {
      p->level_dtype[i] = u8 ? (i == 1 ? FA_F16 : FA_F32) : FA_F64;
      p->in_dtype[i] = u8 ? (p->level_dtype[i] | FA_DTYPE_U8_PYRAMID) : FA_F64;
      const int64_t eb = p->level_dtype[i] == FA_F16 ? 2 : p->level_dtype[i] == FA_F32 ? 4 : 8;
      const int64_t lb = planes * p->H[i] * p->W[i] * eb;
      p->level_x[i] = take(lb);
      p->level_y[i] = take(lb);
    } else {
      p->in_dtype[i] = dtype;
      p->level_dtype[i] = dtype;
    }
    p->pcs[i] = take(planes * p->bpp[i] * 8);
  }
  p->ps_last = take(planes * p->bpp[M - 1] * 8);
  p->scratch = take(static_cast<int64_t>(M) * planes * 8);
  p->total = off;
  return FA_OK;
}

// ---------------------------------------------------------------------------
// Fixed scratch for fa_gpu_ssim_noalloc: the float64 partial sums of one
// call (N * C * slots per plane), in a file-scope device array.  Every GPU the
// library runs on holds its own copy (8 MiB) until the process ends; calls on
// one GPU share it, so calls that overlap on one GPU race.  No slot needs
// clearing: every slot a launch's finalize reads was written by that launch.
constexpr int64_t NOALLOC_SLOTS = FA_NOALLOC_SLOTS;
__device__ __align__(256) double scratch[NOALLOC_SLOTS];

namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<double*> g_scratch[NOALLOC_MAX_DEVICES];

// The device address of the current device's `scratch`, asked once per device
// (hipGetSymbolAddress with that device current) and kept.  The array's name
// is a host-side stand-in in host code and is never passed to a kernel.  The
// lookup may load the code object, which has no place in a graph capture:
// a first call on a device whose stream is capturing gets FA_E_ARG before any
// other HIP call (one eager call on the device must come first).
int scratch_on_current_device(hipStream_t st, double** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -static_cast<int>(e);
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return FA_E_ARG;
  double* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cap);
    if (e != hipSuccess) return -static_cast<int>(e);
    if (cap != hipStreamCaptureStatusNone) return FA_E_ARG;
    void* q = nullptr;
    e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return -static_cast<int>(e);
    if (q == nullptr) return FA_E_INTERNAL;
    p = static_cast<double*>(q);
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return FA_OK;
}

}  // namespace

}  // namespace fa

using namespace fa;

extern "C" {

// No counterpart in the reference: fa_gpu_ssim without the `partial`
// workspace, for callers that cannot allocate (see include/fa_abi.h).
FA_API int fa_gpu_ssim_noalloc(const void* x, const void* y, int dtype, int N, int C, int H,
                               int W, const float* win, int K, double shift, double C1,
                               double C2, float* map_out, double* out_per_image,
                               double* out_total, int device, void* stream) {
  int Hout = 0, Wout = 0;
  int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  const int bpp = ssim_slots(Hout, Wout, K);
  // host-side bound, before any HIP call: the launch below writes
  // N * C * bpp slots of the scratch array
  if (static_cast<int64_t>(N) * C * bpp > NOALLOC_SLOTS) return FA_E_SCRATCH;
  double* partial = nullptr;
  {
    FA_DEVICE_SCOPE(device);
    rc = scratch_on_current_device(static_cast<hipStream_t>(stream), &partial);
    if (rc != FA_OK) return rc;
  }
  return ssim_impl(x, y, dtype, N, C, H, W, nullptr, nullptr, nullptr, win, K, shift, C1, C2,
                   map_out, partial, bpp, out_per_image, out_total, device, stream);
}

// reference: fa_cuda.cu:1158-1165 (fa_cuda_ssim_workspace)
FA_API int fa_gpu_ssim_workspace(int H, int W, int K, int* out_bpp) {
  if (!out_bpp) return FA_E_ARG;
  int Hout = 0, Wout = 0;
  const int rc = ssim_shape(1, 1, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  *out_bpp = ssim_slots(Hout, Wout, K);
  return FA_OK;
}

// reference: fa_cuda.cu:1167-1223 (fa_cuda_ssim)
FA_API int fa_gpu_ssim(const void* x, const void* y, int dtype, int N, int C,
                       int H, int W, const float* win, int K, double shift,
                       double C1, double C2, float* map_out, double* partial,
                       int bpp, double* out_per_image, double* out_total,
                       int device, void* stream) {
  return ssim_impl(x, y, dtype, N, C, H, W, nullptr, nullptr, nullptr, win, K, shift, C1, C2,
                   map_out, partial, bpp, out_per_image, out_total, device, stream);
}

// No counterpart in the reference, which materialises a float32 luma plane
// (functional.py:267-271) and copies crops contiguous (backend.py:346,482).
FA_API int fa_gpu_ssim_ex(const void* x, const void* y, int dtype, int N, int C, int H,
                          int W, const int64_t* x_strides, const int64_t* y_strides,
                          const double* luma, const float* win, int K, double shift,
                          double C1, double C2, float* map_out, double* partial, int bpp,
                          double* out_per_image, double* out_total, int device,
                          void* stream) {
  return ssim_impl(x, y, dtype, N, C, H, W, x_strides, y_strides, luma, win, K, shift, C1, C2,
                   map_out, partial, bpp, out_per_image, out_total, device, stream);
}

// No counterpart in the reference, whose SSIM ends in a finalize launch
// (fa_cuda.cu:1218-1222): fa_gpu_ssim_ex, finished inside the matrix-core
// launch where it can be (include/fa_abi.h states where).
FA_API int fa_gpu_ssim_once(const void* x, const void* y, int dtype, int N, int C, int H,
                            int W, const int64_t* x_strides, const int64_t* y_strides,
                            const double* luma, const float* win, int K, double shift,
                            double C1, double C2, float* map_out, double* partial, int bpp,
                            uint64_t* acc, double* out_per_image, double* out_total,
                            int device, void* stream) {
  return ssim_impl(x, y, dtype, N, C, H, W, x_strides, y_strides, luma, win, K, shift, C1, C2,
                   map_out, partial, bpp, out_per_image, out_total, device, stream, acc);
}

// reference: fa_cuda.cu:1235-1283 (fa_cuda_ssim_cs)
FA_API int fa_gpu_ssim_cs(const void* x, const void* y, int dtype, int N,
                          int C, int H, int W, const float* win, int K,
                          double shift, double C1, double C2, double* partial,
                          double* partial_cs, int bpp, double* out_s,
                          double* out_cs, int device, void* stream) {
  if (!out_s || !out_cs) return FA_E_ARG;
  if (dtype & FA_DTYPE_U8_PYRAMID) return FA_E_DTYPE;  // a hint of the _ex entry only
  return ssim_cs_impl(x, y, dtype, N, C, H, W, nullptr, nullptr, nullptr, win, K, shift, C1,
                      C2, partial, partial_cs, bpp, out_s, out_cs, nullptr, nullptr, nullptr,
                      FA_F64, device, stream);
}

// No counterpart in the reference (it pools between MS-SSIM scales with torch,
// functional.py:876-885, and materialises luma planes and crops).
// fa_gpu_ssim_cs over views with optional luma, plus the next pyramid level.
FA_API int fa_gpu_ssim_cs_ex(const void* x, const void* y, int dtype, int N, int C, int H,
                             int W, const int64_t* x_strides, const int64_t* y_strides,
                             const double* luma, const float* win, int K, double shift,
                             double C1, double C2, double* partial, double* partial_cs,
                             int bpp, double* out_s, double* out_cs, int* out_slots,
                             void* px, void* py, int pool_dtype, int device, void* stream) {
  if (px) {
    // float32 levels hold the pyramid of uint8 input exactly (and so do
    // float16 levels its first level, multiples of 1/4 in [0, 255]); float64
    // levels that of every floating input; a luma plane pools into float64
    const int base = dtype & ~FA_DTYPE_U8_PYRAMID;
    const bool u8p = (dtype & FA_DTYPE_U8_PYRAMID) != 0;
    const bool ok = pool_dtype == FA_F64 ||
                    (pool_dtype == FA_F32 && !luma &&
                     (base == FA_U8 || base == FA_F32 || (u8p && base == FA_F16))) ||
                    (pool_dtype == FA_F16 && !luma && base == FA_U8);
    if (!ok) return FA_E_DTYPE;
  }
  return ssim_cs_impl(x, y, dtype, N, C, H, W, x_strides, y_strides, luma, win, K, shift, C1,
                      C2, partial, partial_cs, bpp, out_s, out_cs, out_slots, px, py, pool_dtype,
                      device, stream);
}

// reference: fa_cuda.cu:1299-1353 (fa_cuda_ssim_backward)
FA_API int fa_gpu_ssim_backward(const float* x, const float* y,
                                const float* dL_dmap, const float* grad_scalar,
                                const float* win, int K, int N, int C, int H,
                                int W, double shift, double C1, double C2,
                                float* aux, float* dx, float* dy, int device,
                                void* stream) {
  if (!x || !y || !win || !aux) return FA_E_ARG;
  if (!dx && !dy) return FA_E_ARG;
  if (!dL_dmap && !grad_scalar) return FA_E_ARG;
  FA_DEVICE_SCOPE(device);
  return ssim_backward_impl<float, MODE_PREP>(x, y, dL_dmap, grad_scalar, nullptr, nullptr,
                                              win, K, N, C, H, W, shift, C1, C2, aux, dx, dy,
                                              nullptr, nullptr, FA_F32, device,
                                              static_cast<hipStream_t>(stream));
}

// reference: fa_cuda.cu:1365-1414 (fa_cuda_ssim_cs_backward)
FA_API int fa_gpu_ssim_cs_backward(const float* x, const float* y,
                                   const float* gs, const float* gcs,
                                   const float* win, int K, int N, int C,
                                   int H, int W, double shift, double C1,
                                   double C2, float* aux, float* dx,
                                   float* dy, int device, void* stream) {
  if (!x || !y || !gs || !gcs || !win || !aux) return FA_E_ARG;
  if (!dx && !dy) return FA_E_ARG;
  FA_DEVICE_SCOPE(device);
  return ssim_backward_impl<float, MODE_PREP_CS>(x, y, nullptr, nullptr, gs, gcs, win, K, N, C,
                                                 H, W, shift, C1, C2, aux, dx, dy,
                                                 nullptr, nullptr, FA_F32, device,
                                                 static_cast<hipStream_t>(stream));
}

// No counterpart in the reference (its MS-SSIM pyramid is float32 and pooled
// by torch).  The fa_gpu_ssim_cs_backward contract for x / y / dx / dy of
// `dtype` FA_F32 or FA_F64 (the exact pyramid levels), plus the gradient of
// the next level that fa_gpu_ssim_cs_ex wrote: gpx / gpy (either may be
// null) of `gp_dtype` FA_F32 or FA_F64, floor(H/2) x floor(W/2) per plane,
// spread as 1/4 over each 2x2 block into dx / dy.  aux stays float32.
FA_API int fa_gpu_ssim_cs_backward_ex(const void* x, const void* y, int dtype,
                                      const float* gs, const float* gcs,
                                      const float* win, int K, int N, int C,
                                      int H, int W, double shift, double C1,
                                      double C2, const void* gpx, const void* gpy,
                                      int gp_dtype, float* aux, void* dx,
                                      void* dy, int device, void* stream) {
  if (!x || !y || !gs || !gcs || !win || !aux) return FA_E_ARG;
  if (!dx && !dy) return FA_E_ARG;
  if (dtype != FA_F32 && dtype != FA_F64) return FA_E_DTYPE;
  if ((gpx || gpy) && gp_dtype != FA_F32 && gp_dtype != FA_F64) return FA_E_DTYPE;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FA_F32)
    return ssim_backward_impl<float, MODE_PREP_CS>(
        static_cast<const float*>(x), static_cast<const float*>(y), nullptr, nullptr, gs, gcs,
        win, K, N, C, H, W, shift, C1, C2, aux, static_cast<float*>(dx),
        static_cast<float*>(dy), gpx, gpy, gp_dtype, device, st);
  return ssim_backward_impl<double, MODE_PREP_CS>(
      static_cast<const double*>(x), static_cast<const double*>(y), nullptr, nullptr, gs, gcs,
      win, K, N, C, H, W, shift, C1, C2, aux, static_cast<double*>(dx),
      static_cast<double*>(dy), gpx, gpy, gp_dtype, device, st);
}

// No counterpart in the reference, whose MS-SSIM training path runs the CS
// forward of every scale and, in the backward, a coefficient pass before the
// scatter (fa_cuda.cu:655-784 per scale).  MS-SSIM's loss reads one plane
// mean per scale (cs below the coarsest, SSIM there), so this CS pass in
// float64 also writes the coefficient maps for a unit gradient of that mean
// (unit_s: of the SSIM means, else of the cs means); fa_gpu_ssim_cs_scatter
// then scales them by each plane's upstream gradient.
FA_API int fa_gpu_ssim_cs_coef(const void* x, const void* y, int dtype, int N, int C, int H,
                               int W, const float* win, int K, double shift, double C1,
                               double C2, int unit_s, double* partial, double* partial_cs,
                               int bpp, double* out_s, double* out_cs, void* px, void* py,
                               int pool_dtype, float* aux, int aux_dy, int device,
                               void* stream) {
  if (!x || !y || !win || !partial || !partial_cs || !out_s || !out_cs || !aux)
    return FA_E_ARG;
  if (dtype != FA_F32 && dtype != FA_F64) return FA_E_DTYPE;
  if ((px == nullptr) != (py == nullptr)) return FA_E_ARG;
  if (px && pool_dtype != FA_F32 && pool_dtype != FA_F64) return FA_E_DTYPE;
  int Hout = 0, Wout = 0;
  int rc = ssim_shape(N, C, H, W, K, &Hout, &Wout);
  if (rc != FA_OK) return rc;
  if (bpp != ssim_slots(Hout, Wout, K)) return FA_E_ARG;
  SsimArgs a = {};
  rc = set_views(a, C, H, W, nullptr, nullptr, nullptr);
  if (rc != FA_OK) return rc;
  const int64_t planes = static_cast<int64_t>(N) * C;
  const int64_t npix = static_cast<int64_t>(Hout) * Wout;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  a.x = x;
  a.y = y;
  a.H = H;
  a.W = W;
  a.Hout = Hout;
  a.Wout = Wout;
  a.shift = shift;
  a.C1 = C1;
  a.C2 = C2;
  a.win = win;
  a.partial = partial;
  a.partial_cs = partial_cs;
  a.px = px;
  a.py = py;
  a.pool_f64 = pool_dtype == FA_F64 ? 1 : 0;
  a.gnorm = 1.0 / static_cast<double>(npix);
  a.unit_s = unit_s ? 1 : 0;
  a.ob = aux;
  a.oc = aux + planes * npix;
  a.otx = aux + 2 * planes * npix;
  a.oty = aux_dy ? aux + 3 * planes * npix : nullptr;
  rc = dtype == FA_F32 ? launch_ssim_k<float, double, MODE_CSF>(K, a, planes, device, st)
                       : launch_ssim_k<double, double, MODE_CSF>(K, a, planes, device, st);
  if (rc != FA_OK) return rc;
  hipLaunchKernelGGL(planes2_kernel, dim3(static_cast<unsigned>(planes)), dim3(BLOCK), 0, st,
                     partial, partial_cs, a.bpp, static_cast<double>(npix), out_s, out_cs);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// No counterpart in the reference (see fa_gpu_ssim_cs_coef): the scatter of
// that pass's maps `aux`, times gscale[plane] (the plane mean's upstream
// gradient, N * C float32), plus a quarter of the pyramid level's gradient
// (gpx / gpy of gp_dtype, either may be null) over each 2x2 block.
FA_API int fa_gpu_ssim_cs_scatter(const void* x, const void* y, int dtype, const double* gscale,
                                  const float* win, int K, int N, int C, int H, int W,
                                  double shift, const float* aux, int aux_dy, const void* gpx,
                                  const void* gpy, int gp_dtype, void* dx, void* dy, int device,
                                  void* stream) {
  if (!x || !y || !gscale || !win || !aux) return FA_E_ARG;
  if (!dx && !dy) return FA_E_ARG;
  if (dy && !aux_dy) return FA_E_ARG;
  if (dtype != FA_F32 && dtype != FA_F64) return FA_E_DTYPE;
  if ((gpx || gpy) && gp_dtype != FA_F32 && gp_dtype != FA_F64) return FA_E_DTYPE;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FA_F32)
    return scatter_impl<float>(static_cast<const float*>(x), static_cast<const float*>(y), gscale,
                               win, K, N, C, H, W, shift, aux, aux_dy != 0, gpx, gpy, gp_dtype,
                               static_cast<float*>(dx), static_cast<float*>(dy), device, st);
  return scatter_impl<double>(static_cast<const double*>(x), static_cast<const double*>(y),
                              gscale, win, K, N, C, H, W, shift, aux, aux_dy != 0, gpx, gpy,
                              gp_dtype, static_cast<double*>(dx), static_cast<double*>(dy),
                              device, st);
}

// No counterpart in the reference, which reduces each MS-SSIM scale in its own
// finalize launch and combines the scales with torch ops (functional.py:897-901).
FA_API int fa_gpu_ms_ssim_reduce(const double* const* partials, const int* slots,
                                 const double* npix, const double* weights, int M, int N,
                                 int C, double* plane_scratch, double* out_per_image,
                                 double* out_total, int device, void* stream) {
  return ms_reduce_impl(partials, slots, npix, weights, M, N, C, plane_scratch, out_per_image,
                        out_total, device, stream);
}

// Checks and packs fa_gpu_ms_ssim_head(_backward)'s scale arrays.
static int ms_head_args(const double* const* terms, const double* weights, int M, int N, int C,
                        MsHead* h) {
  if (!terms || !weights) return FA_E_ARG;
  if (M <= 0 || M > MS_MAX_SCALES || N <= 0 || C <= 0) return FA_E_SHAPE;
  if (static_cast<int64_t>(N) * C > static_cast<int64_t>(INT32_MAX) - BLOCK) return FA_E_SHAPE;
  *h = MsHead{};
  for (int m = 0; m < M; ++m) {
    if (!terms[m]) return FA_E_ARG;
    h->t[m] = terms[m];
    h->w[m] = weights[m];
  }
  h->M = M;
  h->N = N;
  h->C = C;
  return FA_OK;
}

// No counterpart in the reference, which combines the MS-SSIM scales with
// torch ops (functional.py:897-901): about six launches forward and twenty
// backward per training step, here one each.
FA_API int fa_gpu_ms_ssim_head(const double* const* terms, int M, int N, int C,
                               const double* weights, double* out_per_image, double* out_total,
                               int device, void* stream) {
  MsHead h;
  const int rc = ms_head_args(terms, weights, M, N, C, &h);
  if (rc != FA_OK) return rc;
  if (!out_per_image && !out_total) return FA_E_ARG;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ms_head_kernel, dim3(1), dim3(BLOCK), 0, st, h, out_per_image, out_total);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// No counterpart in the reference (see fa_gpu_ms_ssim_head).
FA_API int fa_gpu_ms_ssim_head_backward(const double* const* terms, int M, int N, int C,
                                        const double* weights, const double* g_per_image,
                                        const double* g_total, double* const* g_terms,
                                        int device, void* stream) {
  MsHead h;
  const int rc = ms_head_args(terms, weights, M, N, C, &h);
  if (rc != FA_OK) return rc;
  if (!g_terms || (g_per_image == nullptr) == (g_total == nullptr)) return FA_E_ARG;
  MsHeadGrads g = {};
  for (int m = 0; m < M; ++m) g.g[m] = g_terms[m];
  const int64_t planes = static_cast<int64_t>(N) * C;
  FA_DEVICE_SCOPE(device);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ms_head_backward_kernel,
                     dim3(static_cast<unsigned>((planes + MS_HEAD_BW_PLANES - 1) / MS_HEAD_BW_PLANES)),
                     dim3(BLOCK), 0, st, h, g_per_image, g_total, g);
  FA_LAUNCH_CHECK();
  return FA_OK;
}

// No counterpart in the reference, whose MS-SSIM is a Python loop over the
// scales with torch pooling between them (functional.py:874-901).  The
// workspace of one fa_gpu_ms_ssim call.
FA_API int fa_gpu_ms_ssim_workspace(int dtype, int N, int C, int H, int W, int K, int M,
                                    int luma, int64_t* out_bytes) {
  if (!out_bytes) return FA_E_ARG;
  MsPlan p;
  const int rc = ms_plan(dtype, N, C, H, W, K, M, luma != 0, &p);
  if (rc != FA_OK) return rc;
  *out_bytes = p.total;
  return FA_OK;
}

// No counterpart in the reference (see fa_gpu_ms_ssim_workspace): the whole
// inference MS-SSIM in one call -- every scale's fused CS pass (which also
// writes the next pyramid level) and the reduction, launched back to back.
FA_API int fa_gpu_ms_ssim(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                          const int64_t* x_strides, const int64_t* y_strides,
                          const double* luma, const float* win, int K, double shift,
                          double C1, double C2, const double* weights, int M, void* workspace,
                          int64_t workspace_bytes, uint64_t* acc, double* out_per_image,
                          double* out_total, int device, void* stream) {
  if (!x || !y || !win || !weights || !workspace) return FA_E_ARG;
  if (!out_per_image && !out_total) return FA_E_ARG;
  if (luma && C != 3) return FA_E_SHAPE;
  MsPlan p;
  int rc = ms_plan(dtype, N, C, H, W, K, M, luma != nullptr, &p);
  if (rc != FA_OK) return rc;
  if (workspace_bytes < p.total) return FA_E_ARG;
  char* ws = static_cast<char*>(workspace);
  if (acc && dtype == FA_U8 && !luma) {
    // three launches, the reduction finished in the last (ssim_mfma_ms)
    SsimArgs v = {};
    rc = set_views(v, C, H, W, x_strides, y_strides, nullptr);
    if (rc != FA_OK) return rc;
    SsimMfmaMs mc = {};
    mc.x = x;
    mc.y = y;
    mc.xsn = v.xsn;
    mc.xsc = v.xsc;
    mc.ysn = v.ysn;
    mc.ysc = v.ysc;
    mc.xsh = v.xsh;
    mc.ysh = v.ysh;
    mc.N = N;
    mc.C = C;
    mc.H = H;
    mc.W = W;
    mc.K = K;
    mc.M = M;
    mc.win = win;
    mc.C1 = C1;
    mc.C2 = C2;
    mc.weights = weights;
    for (int i = 1; i < M; ++i) {
      mc.lx[i] = ws + p.level_x[i];
      mc.ly[i] = ws + p.level_y[i];
    }
    mc.words = acc;
    mc.out_per_image = out_per_image;
    mc.out_total = out_total;
    bool done = false;
    {
      FA_DEVICE_SCOPE(device);
      rc = ssim_mfma_ms(mc, device, static_cast<hipStream_t>(stream), &done);
    }
    if (rc != FA_OK || done) return rc;
  }
  const double* parts[MS_MAX_SCALES];
  int slots[MS_MAX_SCALES];
  double npix[MS_MAX_SCALES];
  for (int i = 0; i < M; ++i) {
    const bool last = i == M - 1;
    const void* xi = i == 0 ? x : ws + p.level_x[i];
    const void* yi = i == 0 ? y : ws + p.level_y[i];
    double* pcs = reinterpret_cast<double*>(ws + p.pcs[i]);
    double* ps = last ? reinterpret_cast<double*>(ws + p.ps_last) : nullptr;
    void* px = last ? nullptr : ws + p.level_x[i + 1];
    void* py = last ? nullptr : ws + p.level_y[i + 1];
    rc = ssim_cs_impl(xi, yi, p.in_dtype[i], N, i == 0 ? C : p.cout, p.H[i], p.W[i],
                      i == 0 ? x_strides : nullptr, i == 0 ? y_strides : nullptr,
                      i == 0 ? luma : nullptr, win, K, shift, C1, C2, ps, pcs, p.bpp[i], nullptr,
                      nullptr, &slots[i], px, py, last ? FA_F64 : p.level_dtype[i + 1], device,
                      stream);
    if (rc != FA_OK) return rc;
    parts[i] = last ? ps : pcs;
    npix[i] = static_cast<double>(p.H[i] - K + 1) * (p.W[i] - K + 1);
  }
  return ms_reduce_impl(parts, slots, npix, weights, M, N, p.cout,
                        reinterpret_cast<double*>(ws + p.scratch), out_per_image, out_total,
                        device, stream);
}

}  // extern "C"
