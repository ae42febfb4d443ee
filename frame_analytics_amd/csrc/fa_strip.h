// The separable-window strip engine behind every SSIM-family kernel.
//
// One workgroup of 256 lanes owns a strip of 256 consecutive *input* columns
// and a chunk of TH output rows of one plane.  Each lane owns exactly one input
// column and walks down it:
//
//   vertical pass (registers).  The lane turns every input row it loads into
//     NP "moment" values and keeps the last RS rows of them in a register ring.
//     Every phase it loads PH new rows and forms the KW-tap vertical sum of
//     PH output rows -- no LDS traffic, no bank conflicts, and because the ring
//     slot of every row is a compile-time constant after unrolling one ring
//     cycle, no register moves either.
//
//   horizontal pass (LDS).  The PH x NP vertical sums of all 256 columns go to
//     one of two LDS buffers; after a single barrier wave i takes phase row i
//     and lane g takes output columns 4g..4g+3, reading the 16 values it needs
//     per plane with ds_read_b128 (consecutive lanes, consecutive 16-byte
//     chunks: conflict free).  Double buffering means one barrier per phase.
//
// A strip yields 256 - (KW-1) output columns; neighbouring strips overlap by
// KW-1 input columns, and neighbouring row chunks by KW-1 input rows.
//
// What the lane loads (Pol::set_column once, Pol::load(row) per row; loads are
// branch free, out-of-grid rows and columns are clamped or zeroed by the
// policy), what it does with each raw row besides (Pol::pool: the MS-SSIM
// pyramid step rides along, one (even, odd) row pair at a time), which
// moments it forms and what happens to each output pixel (Pol::emit with a
// validity flag and what Pol::emit_load fetched for it a phase earlier,
// Pol::end_row after each lane's four) is a policy (see fa_ssim.hip): the SSIM forward (4 moments, float32 or
// float64), the backward coefficient pass, and the backward scatter (the
// coefficient maps filtered back onto the full grid, which is the same
// correlation with the input origin moved back by KW-1 and zero padding).
#pragma once

#include "fa_common.h"
#include "fa_widen.h"

namespace fa {

constexpr int STRIP_COLS = BLOCK;  // input columns per workgroup, one per lane
constexpr int PH = WAVES_PER_BLOCK;  // output rows per phase: one per wave
constexpr int HROW = STRIP_COLS + 16;  // LDS row pitch, room for the last 16-wide read
constexpr int COLS_PER_LANE = 4;       // horizontal outputs per lane per phase

template <int KW>
struct StripGeom {
  static constexpr int OUTW = STRIP_COLS - (KW - 1);        // output columns per strip
  static constexpr int RS = ((KW - 1 + PH + PH - 1) / PH) * PH;  // ring rows
  static constexpr int NCYC = RS / PH;                        // phases per ring cycle
};

// Strip / chunk counts of an out_H x out_W output grid.
inline void strip_grid(int out_H, int out_W, int K, int TH, int* strips, int* chunks) {
  const int outw = STRIP_COLS - (K - 1);
  *strips = (out_W + outw - 1) / outw;
  *chunks = (out_H + TH - 1) / TH;
}

template <typename CT>
struct LdsVec;  // 16-byte LDS vector of CT
template <> struct LdsVec<float> { using type = float4; static constexpr int N = 4; };
template <> struct LdsVec<double> { using type = double2; static constexpr int N = 2; };

// Runs the whole strip for one (plane, strip, chunk) workgroup.
//   off        : input row/column of tap 0 for output (0, 0): 0 for a valid
//                correlation, -(KW-1) for the transposed (scatter) one
//   out_H,out_W: output grid (the policy knows its input grid)
template <class Pol, int KW>
__device__ inline void strip_engine(Pol& pol, const float* __restrict__ win,
                                    int off, int out_H, int out_W, int TH,
                                    int strip, int chunk,
                                    typename Pol::CT (*sbuf)[PH][Pol::NP / Pol::NSUB][HROW]) {
  using CT = typename Pol::CT;
  using Raw = typename Pol::Raw;
  constexpr int NP = Pol::NP;
  constexpr int NSUB = Pol::NSUB;  // LDS sub-phases per phase
  constexpr int NPL = NP / NSUB;   // moments per sub-phase
  static_assert(NP % NSUB == 0, "sub-phases split the moments evenly");
  constexpr int OUTW = StripGeom<KW>::OUTW;
  constexpr int RS = StripGeom<KW>::RS;
  constexpr int NCYC = StripGeom<KW>::NCYC;
  using V16 = typename LdsVec<CT>::type;
  constexpr int VN = LdsVec<CT>::N;
  constexpr int NREAD = 16 / VN;  // 16-byte LDS reads per plane per lane

  // float64 taps take their weights from scalar registers (22 vector
  // registers fewer): widen_uniform converts on the scalar unit.
  CT w[KW];
#pragma unroll
  for (int j = 0; j < KW; ++j) {
    if constexpr (sizeof(CT) == 8) w[j] = widen_uniform(win[j]);
    else w[j] = static_cast<CT>(win[j]);
  }

  const int lane = threadIdx.x;
  const int col0 = strip * OUTW;          // first output column of the strip
  const int in_col = col0 + off + lane;   // this lane's input column
  const int r0 = chunk * TH;              // first output row of the chunk
  const int rows_here = min(TH, out_H - r0);
  const int in_row0 = r0 + off;           // input row of tap 0 for output row r0
  const int nph = (rows_here + PH - 1) / PH;

  // The column is per lane and fixed for the whole strip; the row is uniform
  // across the workgroup, so every row address is scalar arithmetic and a load
  // costs one 32-bit lane offset.
  pol.set_column(in_col);

  // Rows come in (even, odd) pairs for Pol::pool2: KW - 1 and PH are even,
  // and the forward's in_row0 (a chunk origin) is even.
  static_assert(KW % 2 == 1 && PH % 2 == 0, "row pairs must not straddle a phase");
  // The ring holds what the policy keeps per input row (Pol::NR values of
  // Pol::RT; Pol::moments fills a row, Pol::vtap adds one tap's weighted
  // moments of sub-phase s): the NP moments themselves, or fewer, narrower
  // values the tap expands exactly, which frees registers for the float64
  // kernels.
  using RT = typename Pol::RT;
  constexpr int NR = Pol::NR;
  RT ring[RS][NR];
#pragma unroll
  for (int i = 0; i < KW - 1; i += 2) {
    const Raw ra = pol.load(in_row0 + i);
    const Raw rb = pol.load(in_row0 + i + 1);
    pol.pool2(in_row0 + i, ra, rb);
    pol.moments(ra, ring[i]);
    pol.moments(rb, ring[i + 1]);
  }

  Raw pend[PH];
#pragma unroll
  for (int i = 0; i < PH; ++i) pend[i] = pol.load(in_row0 + KW - 1 + i);

  // phase row of this wave, in a scalar register: the row of every output a
  // wave emits is uniform, so a policy can address its output row with a
  // scalar buffer resource
  const int hrow = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
  const int oc_l = COLS_PER_LANE * (threadIdx.x % WAVE);  // strip-local output column

  // What emit reads from memory for the lane's outputs (Pol::EIn: the input
  // samples of the scatter, an upstream gradient map) is loaded one phase
  // ahead, so its latency hides behind the next phase's vertical taps
  // instead of stalling the horizontal pass.  Pol::emit_load clamps its
  // addresses into the grid; rows and columns past it are never emitted.
  using EIn = typename Pol::EIn;
  static_assert(OUTW % 2 == 0, "a lane's first output column is even");
  EIn ein = pol.emit_load(r0 + hrow, col0 + oc_l);

  for (int qc = 0; qc < nph; qc += NCYC) {
#pragma unroll
    for (int u = 0; u < NCYC; ++u) {
      const int q = qc + u;
      if (q < nph) {  // uniform across the workgroup
#pragma unroll
        for (int i = 0; i < PH; i += 2) pol.pool2(in_row0 + KW - 1 + q * PH + i, pend[i], pend[i + 1]);
#pragma unroll
        for (int i = 0; i < PH; ++i) pol.moments(pend[i], ring[(KW - 1 + u * PH + i) % RS]);
        // Prefetch the next phase unconditionally: loads are clamped by the
        // policy, and a guard here would cost register copies every phase.
#pragma unroll
        for (int i = 0; i < PH; ++i) pend[i] = pol.load(in_row0 + KW - 1 + (q + 1) * PH + i);

        // The NP moments go through LDS in NSUB sub-phases of NPL each,
        // alternating the two buffers: one barrier per sub-phase.  (The
        // float64 forward splits its four moments in two, which halves its
        // LDS per workgroup and lets more workgroups share a CU.)
        const int orow_l = q * PH + hrow;
        const bool out_lane = orow_l < rows_here && oc_l < OUTW;
        CT h[COLS_PER_LANE][NP];
        EIn ein_next;
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
          // ---- vertical taps, from the register ring --------------------
          // Ring row by ring row: the products a policy forms from a row
          // (the float64 ring keeps x', y' only) are formed once and die at
          // once.  Each output row still adds its taps in the order
          // j = 0 .. KW-1.
          CT (*dst)[NPL][HROW] = sbuf[(q * NSUB + s) & 1];
          CT v[PH][NPL];
#pragma unroll
          for (int i = 0; i < PH; ++i)
#pragma unroll
            for (int p = 0; p < NPL; ++p) v[i][p] = CT(0);
#pragma unroll
          for (int r = 0; r < KW - 1 + PH; ++r) {
#pragma unroll
            for (int i = 0; i < PH; ++i) {
              const int j = r - i;
              if (j >= 0 && j < KW) pol.vtap(w[j], ring[(u * PH + r) % RS], v[i], s);
            }
          }
#pragma unroll
          for (int i = 0; i < PH; ++i)
#pragma unroll
            for (int p = 0; p < NPL; ++p) dst[i][p][lane] = v[i][p];
          if (s == NSUB - 1) ein_next = pol.emit_load(r0 + (q + 1) * PH + hrow, col0 + oc_l);
          __syncthreads();

          // ---- horizontal taps, from LDS --------------------------------
          // Every lane runs them (a lane past the strip's outputs reads
          // columns up to oc_l + 15 < HROW) and every lane emits, with
          // `valid` false where there is no output: the policies' stores are
          // then issued on every path, so the wait for the next phase's loads
          // does not wait for them (a store on some paths only made the
          // compiler wait for every store in flight).
          {
#pragma unroll
            for (int p = 0; p < NPL; ++p) {
              CT in[16];
              const V16* src = reinterpret_cast<const V16*>(&dst[hrow][p][oc_l]);
#pragma unroll
              for (int r = 0; r < NREAD; ++r) {
                const V16 t = src[r];
                __builtin_memcpy(&in[r * VN], &t, sizeof(V16));
              }
#pragma unroll
              for (int k = 0; k < COLS_PER_LANE; ++k) {
                CT a = CT(0);
#pragma unroll
                for (int j = 0; j < KW; ++j) a = fma(w[j], in[k + j], a);
                h[k][s * NPL + p] = a;
              }
            }
          }
        }
        {
          // float64: the sums are formed here, before the emits.  Left to
          // itself the compiler sinks each column's taps into its emit's
          // validity branch, which keeps every plane's 14 LDS values live
          // until the last column (~70 registers more).
          if constexpr (sizeof(CT) == 8) {
#pragma unroll
            for (int k = 0; k < COLS_PER_LANE; ++k)
#pragma unroll
              for (int p = 0; p < NP; ++p) asm volatile("" : "+v"(h[k][p]));
          }
#pragma unroll
          for (int k = 0; k < COLS_PER_LANE; ++k) {
            const int oc = col0 + oc_l + k;
            pol.emit(r0 + orow_l, oc, h[k], out_lane && oc_l + k < OUTW && oc < out_W, ein, k);
          }
          pol.end_row();
        }
        ein = ein_next;
      }
    }
  }
}

}  // namespace fa
