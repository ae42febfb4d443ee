// Host (CPU) kernels behind include/fa_cpu_abi.h: the same metrics as the
// gfx950 library for CPU tensors (reference: frame_analytics/csrc/fa_cpu.cpp,
// whose entry points these replace; the arithmetic follows the same float64
// oracle, the structure is this build's own).
//
//   * one persistent thread pool, serialised: a job is published under a
//     mutex and every worker acknowledges it before run() returns, so calls
//     from several Python threads (ctypes releases the GIL) cannot race and
//     no worker outlives the job it is running
//   * uint8 MSE / L1 are exact: 16-bit differences squared and pair-summed
//     with _mm256_madd_epi16, absolute differences with _mm256_sad_epu8, into
//     int64 per chunk; chunks are combined in a fixed order
//   * SSIM: a task is a band of output rows of one plane; each input row is
//     turned into the four moments x', y', x'y', (x'-y')^2 (x' = x - shift),
//     filtered horizontally into a K-row ring, and every output row is the
//     vertical K-tap sum of the ring -- the formulation of the GPU kernel, in
//     float32 (float64 for float64 input), loops the compiler vectorises
//   * GMSD: bands of output rows, samples and Prewitt sums in float64, and
//     the accumulated quantity is d = 1 - q = (G1-G2)^2 / ((g1+g2)^2 (G1+G2+T))
//     so that the standard deviation does not cancel
#include "fa_cpu_abi.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <thread>
#include <type_traits>
#include <vector>

namespace facpu {

// --------------------------------------------------------------------------
// thread pool
// --------------------------------------------------------------------------
class Pool {
 public:
  static Pool& get() {
    static Pool pool;
    return pool;
  }

  int set_size(int n) {
    std::lock_guard<std::mutex> g(run_mu_);
    if (!started_ && n > 0) want_ = n;
    return size_locked();
  }

  int size() {
    std::lock_guard<std::mutex> g(run_mu_);
    return size_locked();
  }

  // fn(t) for every t in [0, n), on the calling thread and whichever workers
  // join in.  Jobs run one at a time (run_mu_).  A job is one 64-bit ticket,
  // (job id << 32) | next task: a worker claims a task with a compare-and-swap
  // that only succeeds while its job is still the current one, and run()
  // returns once all n tasks have completed -- workers still asleep need not
  // wake for it, and a late one cannot take a task of the next job.
  void run(int64_t n, const std::function<void(int64_t)>& fn) {
    if (n <= 0) return;
    std::lock_guard<std::mutex> g(run_mu_);
    start_locked();
    if (workers_.empty() || n == 1 || n >= (int64_t(1) << 31)) {
      for (int64_t t = 0; t < n; ++t) fn(t);
      return;
    }
    uint32_t id;
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = &fn;
      n_.store(n, std::memory_order_relaxed);
      done_.store(0, std::memory_order_relaxed);
      id = ++job_;
      ticket_.store(static_cast<uint64_t>(id) << 32, std::memory_order_release);
    }
    cv_.notify_all();
    work(id);
    // the last tasks finish within microseconds: spin briefly, then sleep
    auto finished = [&] { return done_.load(std::memory_order_acquire) == n; };
    if (!spin_until(finished)) {
      std::unique_lock<std::mutex> lk(mu_);
      done_cv_.wait(lk, finished);
    }
  }

  ~Pool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_.store(true, std::memory_order_relaxed);
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }

 private:
  Pool() = default;

  // Spin on pred() for up to ~200 microseconds; true if it became true.
  template <typename Pred>
  static bool spin_until(Pred pred) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 1;; ++i) {
      if (pred()) return true;
      _mm_pause();
      if ((i & 255) == 0 &&
          std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200))
        return pred();
    }
  }

  int size_locked() const {
    if (started_) return static_cast<int>(workers_.size()) + 1;
    return want_ > 0 ? want_ : default_size();
  }

  static int default_size() {
    const unsigned hc = std::thread::hardware_concurrency();
    return hc > 0 ? static_cast<int>(hc) : 1;
  }

  void start_locked() {
    if (started_) return;
    started_ = true;
    const int n = (want_ > 0 ? want_ : default_size()) - 1;
    for (int i = 0; i < n; ++i) workers_.emplace_back([this] { worker(); });
  }

  // Claims and runs tasks of job `id` until none is left.  fn_ and n_ are
  // read only after a successful claim: the job cannot complete (so no later
  // job can overwrite them) while a claimed task is outstanding.
  void work(uint32_t id) {
    uint64_t t = ticket_.load(std::memory_order_acquire);
    for (;;) {
      if (static_cast<uint32_t>(t >> 32) != id) return;
      const int64_t idx = static_cast<int64_t>(t & 0xffffffffu);
      const int64_t n = n_.load(std::memory_order_relaxed);
      if (idx >= n) return;
      if (!ticket_.compare_exchange_weak(t, t + 1, std::memory_order_acq_rel,
                                         std::memory_order_acquire))
        continue;  // t now holds the current ticket
      (*fn_)(idx);
      if (done_.fetch_add(1, std::memory_order_acq_rel) + 1 == n) {
        std::lock_guard<std::mutex> lk(mu_);  // pairs with the waiter's predicate check
        done_cv_.notify_all();
      }
      t = ticket_.load(std::memory_order_acquire);
    }
  }

  void worker() {
    uint32_t seen = 0;
    auto fresh = [&] {
      return stop_.load(std::memory_order_relaxed) ||
             static_cast<uint32_t>(ticket_.load(std::memory_order_acquire) >> 32) != seen;
    };
    for (;;) {
      if (!spin_until(fresh)) {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, fresh);
      }
      if (stop_.load(std::memory_order_relaxed)) return;
      seen = static_cast<uint32_t>(ticket_.load(std::memory_order_acquire) >> 32);
      work(seen);
    }
  }

  std::mutex run_mu_;  // one job at a time
  std::mutex mu_;      // pairs with the condition variables
  std::condition_variable cv_, done_cv_;
  std::vector<std::thread> workers_;
  const std::function<void(int64_t)>* fn_ = nullptr;  // published before the ticket
  std::atomic<int64_t> n_{0};  // a stale read is harmless: the claim's CAS decides
  uint32_t job_ = 0;
  std::atomic<uint64_t> ticket_{0};
  std::atomic<int64_t> done_{0};
  std::atomic<bool> stop_{false};
  bool started_ = false;
  int want_ = 0;
};

// --------------------------------------------------------------------------
// element types
// --------------------------------------------------------------------------
struct half_t { uint16_t bits; };
struct bf16_t { uint16_t bits; };

// IEEE binary16 -> binary32, all classes (normal, subnormal, inf, nan).
inline float half_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0x1fu) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  } else if (mant == 0) {
    bits = sign;
  } else {  // subnormal: normalise
    int e = -1;
    do {
      ++e;
      mant <<= 1;
    } while ((mant & 0x400u) == 0);
    bits = sign | ((112u - static_cast<uint32_t>(e)) << 23) | ((mant & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

template <typename T> inline double to_d(T v) { return static_cast<double>(v); }
template <> inline double to_d<half_t>(half_t v) { return half_to_float(v.bits); }
template <> inline double to_d<bf16_t>(bf16_t v) {
  const uint32_t bits = static_cast<uint32_t>(v.bits) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Element -> compute type; integers and floats convert directly, the 16-bit
// floats through their exact float32 value.
template <typename CT, typename T>
inline CT to_c(T v) {
  if constexpr (std::is_arithmetic<T>::value) {
    return static_cast<CT>(v);
  } else {
    return static_cast<CT>(static_cast<float>(to_d(v)));
  }
}

// Row sums widened to float64 lanes: (sum a, sum b) or, with SQ, (sum a,
// sum a^2).  The AVX2 lanes keep every addition in float64.
inline __m256d lo_pd(__m256 v) { return _mm256_cvtps_pd(_mm256_castps256_ps128(v)); }
inline __m256d hi_pd(__m256 v) { return _mm256_cvtps_pd(_mm256_extractf128_ps(v, 1)); }
inline double hsum(__m256d v) {
  alignas(32) double l[4];
  _mm256_store_pd(l, v);
  return (l[0] + l[1]) + (l[2] + l[3]);
}

template <bool SQ>
inline void row_sums(const float* a, const float* b, int n, double* sa, double* sb) {
  __m256d x0 = _mm256_setzero_pd(), x1 = x0, y0 = x0, y1 = x0;
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    const __m256 va = _mm256_loadu_ps(a + c);
    const __m256d al = lo_pd(va), ah = hi_pd(va);
    x0 = _mm256_add_pd(x0, al);
    x1 = _mm256_add_pd(x1, ah);
    if constexpr (SQ) {
      y0 = _mm256_fmadd_pd(al, al, y0);
      y1 = _mm256_fmadd_pd(ah, ah, y1);
    } else {
      const __m256 vb = _mm256_loadu_ps(b + c);
      y0 = _mm256_add_pd(y0, lo_pd(vb));
      y1 = _mm256_add_pd(y1, hi_pd(vb));
    }
  }
  double ra = hsum(_mm256_add_pd(x0, x1)), rb = hsum(_mm256_add_pd(y0, y1));
  for (; c < n; ++c) {
    const double v = a[c];
    ra += v;
    rb += SQ ? v * v : static_cast<double>(b[c]);
  }
  *sa += ra;
  *sb += rb;
}

template <bool SQ>
inline void row_sums(const double* a, const double* b, int n, double* sa, double* sb) {
  __m256d x0 = _mm256_setzero_pd(), x1 = x0, y0 = x0, y1 = x0;
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    const __m256d a0 = _mm256_loadu_pd(a + c), a1 = _mm256_loadu_pd(a + c + 4);
    x0 = _mm256_add_pd(x0, a0);
    x1 = _mm256_add_pd(x1, a1);
    if constexpr (SQ) {
      y0 = _mm256_fmadd_pd(a0, a0, y0);
      y1 = _mm256_fmadd_pd(a1, a1, y1);
    } else {
      y0 = _mm256_add_pd(y0, _mm256_loadu_pd(b + c));
      y1 = _mm256_add_pd(y1, _mm256_loadu_pd(b + c + 4));
    }
  }
  double ra = hsum(_mm256_add_pd(x0, x1)), rb = hsum(_mm256_add_pd(y0, y1));
  for (; c < n; ++c) {
    ra += a[c];
    rb += SQ ? a[c] * a[c] : b[c];
  }
  *sa += ra;
  *sb += rb;
}

// Sum of n values in float64 lanes.
inline double lane_sum(const float* a, int n) {
  __m256d x0 = _mm256_setzero_pd(), x1 = x0;
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    const __m256 v = _mm256_loadu_ps(a + c);
    x0 = _mm256_add_pd(x0, lo_pd(v));
    x1 = _mm256_add_pd(x1, hi_pd(v));
  }
  double r = hsum(_mm256_add_pd(x0, x1));
  for (; c < n; ++c) r += a[c];
  return r;
}

inline double lane_sum(const double* a, int n) {
  __m256d x0 = _mm256_setzero_pd(), x1 = x0;
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    x0 = _mm256_add_pd(x0, _mm256_loadu_pd(a + c));
    x1 = _mm256_add_pd(x1, _mm256_loadu_pd(a + c + 4));
  }
  double r = hsum(_mm256_add_pd(x0, x1));
  for (; c < n; ++c) r += a[c];
  return r;
}

// --------------------------------------------------------------------------
// pixel reductions
// --------------------------------------------------------------------------
constexpr int64_t PIX_CHUNK = int64_t(1) << 15;  // elements per task: 24 tasks at 1x3x512x512

// Exact sum of (a-b)^2 of n uint8 pairs: |a-b| from two saturating
// subtractions, widened to 16 bits in-lane and squared + pair-summed by madd.
inline uint64_t sse_u8(const uint8_t* a, const uint8_t* b, int64_t n) {
  uint64_t total = 0;
  int64_t i = 0;
  const __m256i zero = _mm256_setzero_si256();
  while (i + 32 <= n) {
    // each 32-bit lane gains at most 2 * 255^2 per step; 2048 steps stay < 2^31
    __m256i acc0 = zero, acc1 = zero;
    const int64_t stop = std::min(n, i + int64_t(2048) * 32);
    for (; i + 32 <= stop; i += 32) {
      const __m256i va = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(a + i));
      const __m256i vb = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(b + i));
      const __m256i d = _mm256_or_si256(_mm256_subs_epu8(va, vb), _mm256_subs_epu8(vb, va));
      const __m256i lo = _mm256_unpacklo_epi8(d, zero);
      const __m256i hi = _mm256_unpackhi_epi8(d, zero);
      acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(lo, lo));
      acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(hi, hi));
    }
    alignas(32) int32_t lanes[16];
    _mm256_store_si256(reinterpret_cast<__m256i*>(lanes), acc0);
    _mm256_store_si256(reinterpret_cast<__m256i*>(lanes + 8), acc1);
    for (int k = 0; k < 16; ++k) total += static_cast<uint64_t>(static_cast<uint32_t>(lanes[k]));
  }
  for (; i < n; ++i) {
    const int d = static_cast<int>(a[i]) - static_cast<int>(b[i]);
    total += static_cast<uint64_t>(d * d);
  }
  return total;
}

// Exact sum of |a-b| of n uint8 pairs.
inline uint64_t sad_u8(const uint8_t* a, const uint8_t* b, int64_t n) {
  __m256i acc = _mm256_setzero_si256();
  int64_t i = 0;
  for (; i + 32 <= n; i += 32) {
    const __m256i va = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(a + i));
    const __m256i vb = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(b + i));
    acc = _mm256_add_epi64(acc, _mm256_sad_epu8(va, vb));
  }
  alignas(32) uint64_t lanes[4];
  _mm256_store_si256(reinterpret_cast<__m256i*>(lanes), acc);
  uint64_t total = lanes[0] + lanes[1] + lanes[2] + lanes[3];
  for (; i < n; ++i) total += static_cast<uint64_t>(a[i] > b[i] ? a[i] - b[i] : b[i] - a[i]);
  return total;
}

// The four penalties (reference fa_cpu.cpp pix_term, fa_cuda.cu:252-260):
// float32 for Charbonnier below float64 input, float64 otherwise.
template <int OP, typename A>
inline A pix_term(A d, A p) {
  if constexpr (OP == FA_OP_MSE) {
    return d * d;
  } else if constexpr (OP == FA_OP_L1) {
    return d < A(0) ? -d : d;
  } else if constexpr (OP == FA_OP_CHARB) {
    return std::sqrt(d * d + p);
  } else {
    const A a = d < A(0) ? -d : d;
    const A lo = a < p ? a : p;
    return A(0.5) * lo * lo + p * (a - lo);
  }
}

constexpr int PIX_BLOCK = 1024;  // terms per vectorised block

// A block of terms (the exact difference rounded once to A), out of line so
// that the loop keeps its no-alias facts and vectorises.
template <typename T, int OP, typename A>
__attribute__((noinline)) void pix_terms(const T* __restrict__ a, const T* __restrict__ b, int n,
                                         A p, A* __restrict__ out) {
  for (int i = 0; i < n; ++i) {
    if constexpr (std::is_same<T, uint8_t>::value) {
      out[i] = pix_term<OP, A>(static_cast<A>(static_cast<int>(a[i]) - static_cast<int>(b[i])), p);
    } else {
      out[i] = pix_term<OP, A>(static_cast<A>(to_d(a[i]) - to_d(b[i])), p);
    }
  }
}

// Terms are evaluated in A (float32 only for Charbonnier below float64 input)
// and always summed in float64 lanes.
template <typename T, int OP>
double float_sum(const T* a, const T* b, int64_t n, double param) {
  constexpr bool WIDE = OP != FA_OP_CHARB || std::is_same<T, double>::value;
  using A = typename std::conditional<WIDE, double, float>::type;
  const A p = static_cast<A>(param);
  alignas(32) A buf[PIX_BLOCK];
  double acc = 0.0;
  for (int64_t i0 = 0; i0 < n; i0 += PIX_BLOCK) {
    const int m = static_cast<int>(std::min<int64_t>(PIX_BLOCK, n - i0));
    pix_terms<T, OP, A>(a + i0, b + i0, m, p, buf);
    acc += lane_sum(buf, m);
  }
  return acc;
}

template <typename T>
double chunk_sum(int op, const void* va, const void* vb, int64_t off, int64_t n, double param,
                 bool* exact, uint64_t* isum) {
  const T* a = static_cast<const T*>(va) + off;
  const T* b = static_cast<const T*>(vb) + off;
  if constexpr (std::is_same<T, uint8_t>::value) {
    if (op == FA_OP_MSE) {
      *exact = true;
      *isum = sse_u8(a, b, n);
      return 0.0;
    }
    if (op == FA_OP_L1) {
      *exact = true;
      *isum = sad_u8(a, b, n);
      return 0.0;
    }
    *exact = false;
    return op == FA_OP_CHARB ? float_sum<uint8_t, FA_OP_CHARB>(a, b, n, param)
                             : float_sum<uint8_t, FA_OP_HUBER>(a, b, n, param);
  } else {
    *exact = false;
    switch (op) {
      case FA_OP_MSE: return float_sum<T, FA_OP_MSE>(a, b, n, param);
      case FA_OP_L1: return float_sum<T, FA_OP_L1>(a, b, n, param);
      case FA_OP_CHARB: return float_sum<T, FA_OP_CHARB>(a, b, n, param);
      default: return float_sum<T, FA_OP_HUBER>(a, b, n, param);
    }
  }
}

// --------------------------------------------------------------------------
// SSIM
// --------------------------------------------------------------------------
constexpr int SSIM_BAND = 32;  // output rows per task

template <typename T, typename CT>
struct SsimPlane {
  const T* x;
  const T* y;
  int H, W, K;
  const CT* w;  // K taps
  CT shift, C1, C2;
  float* map;   // this plane's map or null
};

// The four moments x', y', x'y', (x'-y')^2 of one input row (x' = x - shift).
// Out of line so that the loop keeps its no-alias facts and vectorises
// (inlined, float32 input ran the scalar copy at twice the whole call's time).
template <typename T, typename CT>
__attribute__((noinline)) void ssim_moments(const T* __restrict__ xr, const T* __restrict__ yr,
                                            int W, CT shift, CT* __restrict__ m0,
                                            CT* __restrict__ m1, CT* __restrict__ m2,
                                            CT* __restrict__ m3) {
  for (int c = 0; c < W; ++c) {
    const CT xs = to_c<CT>(xr[c]) - shift;
    const CT ys = to_c<CT>(yr[c]) - shift;
    const CT d = xs - ys;
    m0[c] = xs;
    m1[c] = ys;
    m2[c] = xs * ys;
    m3[c] = d * d;
  }
}

// dst[c] = sum_j w[j] src[c + j] and dst[c] = sum_j w[j] rows[j][c], c < n:
// each column's K taps accumulate in a register.  Out of line (and ivdep for
// the K row pointers, which GCC would otherwise check pairwise at run time and
// give up on past ten) so that both loops vectorise.
template <int K, typename CT>
__attribute__((noinline)) void filter_h(const CT* __restrict__ src, const CT* __restrict__ w,
                                        int n, CT* __restrict__ dst) {
  for (int c = 0; c < n; ++c) {
    CT acc = w[0] * src[c];
#pragma GCC unroll 11
    for (int j = 1; j < K; ++j) acc = std::fma(w[j], src[c + j], acc);
    dst[c] = acc;
  }
}

template <int K, typename CT>
__attribute__((noinline)) void filter_v(const CT* const* rows, const CT* __restrict__ w, int n,
                                        CT* __restrict__ dst) {
  const CT* r[K];
  for (int j = 0; j < K; ++j) r[j] = rows[j];
#pragma GCC ivdep
  for (int c = 0; c < n; ++c) {
    CT acc = w[0] * r[0][c];
#pragma GCC unroll 11
    for (int j = 1; j < K; ++j) acc = std::fma(w[j], r[j][c], acc);
    dst[c] = acc;
  }
}

// Output rows [r0, r1) of one plane; returns the sums of SSIM and cs.  K is a
// compile-time width so that each output column's K taps accumulate in a
// register (one load per tap, one store per column) and the column loops
// vectorise.
template <int K, typename T, typename CT>
void ssim_band(const SsimPlane<T, CT>& P, int r0, int r1, double* out_s, double* out_cs) {
  const int W = P.W, Wout = W - K + 1;
  // ring of K horizontally filtered rows x 4 moments, plus one moments row
  std::vector<CT> ring(static_cast<size_t>(K) * 4 * Wout);
  std::vector<CT> mom(static_cast<size_t>(4) * W);
  std::vector<CT> v(static_cast<size_t>(4) * Wout), sv(static_cast<size_t>(2) * Wout);
  CT w[K];
  for (int j = 0; j < K; ++j) w[j] = P.w[j];
  CT* const m0 = mom.data();
  CT* const m1 = m0 + W;
  CT* const m2 = m1 + W;
  CT* const m3 = m2 + W;
  double sum_s = 0.0, sum_cs = 0.0;
  const CT shift = P.shift, C2 = P.C2;
  const CT k1 = CT(2) * shift * shift + P.C1;

  for (int i = r0; i < r1 + K - 1; ++i) {
    ssim_moments<T, CT>(P.x + static_cast<int64_t>(i) * W, P.y + static_cast<int64_t>(i) * W, W,
                        shift, m0, m1, m2, m3);
    CT* h = ring.data() + static_cast<size_t>((i - r0) % K) * 4 * Wout;
    for (int q = 0; q < 4; ++q)
      filter_h<K, CT>(m0 + static_cast<size_t>(q) * W, w, Wout, h + static_cast<size_t>(q) * Wout);
    const int o = i - (K - 1);  // the output row this input row completes
    if (o < r0) continue;
    for (int q = 0; q < 4; ++q) {
      const CT* rows[K];
      for (int j = 0; j < K; ++j)
        rows[j] = ring.data() + static_cast<size_t>((o + j - r0) % K) * 4 * Wout +
                  static_cast<size_t>(q) * Wout;
      filter_v<K, CT>(rows, w, Wout, v.data() + static_cast<size_t>(q) * Wout);
    }
    const CT* __restrict__ vx = v.data();
    const CT* __restrict__ vy = vx + Wout;
    const CT* __restrict__ vxy = vy + Wout;
    const CT* __restrict__ vdd = vxy + Wout;
    CT* __restrict__ sb = sv.data();
    CT* __restrict__ cb = sb + Wout;
    for (int c = 0; c < Wout; ++c) {
      // A1 = 2 mu_x mu_y + C1, B1 = mu_x^2 + mu_y^2 + C1 (mu = u + shift),
      // A2 = 2 sigma_xy + C2, B2 = sigma_x^2 + sigma_y^2 + C2
      const CT pxy = vx[c] * vy[c];
      const CT du = vx[c] - vy[c];
      const CT A1 = CT(2) * pxy + CT(2) * shift * (vx[c] + vy[c]) + k1;
      const CT B1 = du * du + A1;
      const CT A2 = CT(2) * (vxy[c] - pxy) + C2;
      const CT B2 = vdd[c] + A2 - du * du;
      sb[c] = (A1 * A2) / (B1 * B2);
      cb[c] = A2 / B2;
    }
    if (P.map) {
      float* __restrict__ mrow = P.map + static_cast<int64_t>(o) * Wout;
      for (int c = 0; c < Wout; ++c) mrow[c] = static_cast<float>(sb[c]);
    }
    row_sums<false>(sb, cb, Wout, &sum_s, &sum_cs);
  }
  *out_s = sum_s;
  *out_cs = sum_cs;
}

template <typename T, typename CT>
void ssim_band_k(const SsimPlane<T, CT>& P, int r0, int r1, double* s, double* cs) {
  switch (P.K) {
    case 3: ssim_band<3>(P, r0, r1, s, cs); break;
    case 5: ssim_band<5>(P, r0, r1, s, cs); break;
    case 7: ssim_band<7>(P, r0, r1, s, cs); break;
    case 9: ssim_band<9>(P, r0, r1, s, cs); break;
    default: ssim_band<11>(P, r0, r1, s, cs); break;
  }
}

template <typename T, typename CT>
int ssim_run(const void* x, const void* y, int N, int C, int H, int W, const float* win, int K,
             double shift, double C1, double C2, float* map, double* sums_s, double* sums_cs) {
  const int Hout = H - K + 1, Wout = W - K + 1;
  const int bands = (Hout + SSIM_BAND - 1) / SSIM_BAND;
  const int64_t planes = static_cast<int64_t>(N) * C;
  std::vector<CT> w(K);
  for (int j = 0; j < K; ++j) w[j] = static_cast<CT>(win[j]);
  std::vector<double> ps(static_cast<size_t>(planes) * bands), pcs(ps.size());
  Pool::get().run(planes * bands, [&](int64_t t) {
    const int64_t plane = t / bands;
    const int band = static_cast<int>(t - plane * bands);
    SsimPlane<T, CT> P;
    P.x = static_cast<const T*>(x) + plane * H * W;
    P.y = static_cast<const T*>(y) + plane * H * W;
    P.H = H;
    P.W = W;
    P.K = K;
    P.w = w.data();
    P.shift = static_cast<CT>(shift);
    P.C1 = static_cast<CT>(C1);
    P.C2 = static_cast<CT>(C2);
    P.map = map ? map + plane * Hout * Wout : nullptr;
    const int r0 = band * SSIM_BAND;
    ssim_band_k<T, CT>(P, r0, std::min(Hout, r0 + SSIM_BAND), &ps[t], &pcs[t]);
  });
  for (int64_t p = 0; p < planes; ++p) {  // fixed order: deterministic
    double s = 0.0, cs = 0.0;
    for (int b = 0; b < bands; ++b) {
      s += ps[p * bands + b];
      cs += pcs[p * bands + b];
    }
    sums_s[p] = s;
    if (sums_cs) sums_cs[p] = cs;
  }
  return FA_OK;
}

int ssim_dispatch(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                  const float* win, int K, double shift, double C1, double C2, float* map,
                  double* sums_s, double* sums_cs) {
  switch (dtype) {
    case FA_U8: return ssim_run<uint8_t, float>(x, y, N, C, H, W, win, K, shift, C1, C2, map, sums_s, sums_cs);
    case FA_F16: return ssim_run<half_t, float>(x, y, N, C, H, W, win, K, shift, C1, C2, map, sums_s, sums_cs);
    case FA_BF16: return ssim_run<bf16_t, float>(x, y, N, C, H, W, win, K, shift, C1, C2, map, sums_s, sums_cs);
    case FA_F32: return ssim_run<float, float>(x, y, N, C, H, W, win, K, shift, C1, C2, map, sums_s, sums_cs);
    case FA_F64: return ssim_run<double, double>(x, y, N, C, H, W, win, K, shift, C1, C2, map, sums_s, sums_cs);
    default: return FA_E_DTYPE;
  }
}

int ssim_check(int N, int C, int H, int W, const float* win, int K) {
  if (!win) return FA_E_ARG;
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return FA_E_SHAPE;
  if (K < 3 || K > FA_MAX_WIN || (K & 1) == 0) return FA_E_WINDOW;
  if (H < K || W < K) return FA_E_SHAPE;
  return FA_OK;
}

// --------------------------------------------------------------------------
// GMSD
// --------------------------------------------------------------------------
constexpr int GMSD_BAND = 32;   // output rows per task
constexpr int GMSD_COLS = 512;  // output columns per task: the rows stay in L1

// One sampled row pair (2x2 means when downsampling) as its sum x + y and
// difference x - y in CT.  Kept out of line: inlined into the band loop, GCC
// loses the no-alias facts and runs the scalar copy of this loop (measured
// 2.6x slower overall).
template <typename T, typename CT>
__attribute__((noinline)) void gmsd_row(const T* __restrict__ x, const T* __restrict__ y, int W,
                                        int Wd, bool down, int r, CT* __restrict__ sum,
                                        CT* __restrict__ dif) {
  // x, y point at the tile's first input column; Wd samples are read
  if (down) {
    const T* x0 = x + static_cast<int64_t>(2 * r) * W;
    const T* x1 = x0 + W;
    const T* y0 = y + static_cast<int64_t>(2 * r) * W;
    const T* y1 = y0 + W;
    // differences before the mean: x - y of two close values is exact, the
    // difference of two rounded means would not be
    for (int c = 0; c < Wd; ++c) {
      const CT a0 = to_c<CT>(x0[2 * c]), a1 = to_c<CT>(x0[2 * c + 1]);
      const CT a2 = to_c<CT>(x1[2 * c]), a3 = to_c<CT>(x1[2 * c + 1]);
      const CT b0 = to_c<CT>(y0[2 * c]), b1 = to_c<CT>(y0[2 * c + 1]);
      const CT b2 = to_c<CT>(y1[2 * c]), b3 = to_c<CT>(y1[2 * c + 1]);
      sum[c] = CT(0.25) * (((a0 + b0) + (a1 + b1)) + ((a2 + b2) + (a3 + b3)));
      dif[c] = CT(0.25) * (((a0 - b0) + (a1 - b1)) + ((a2 - b2) + (a3 - b3)));
    }
  } else {
    const T* x0 = x + static_cast<int64_t>(r) * W;
    const T* y0 = y + static_cast<int64_t>(r) * W;
    for (int c = 0; c < Wd; ++c) {
      const CT a = to_c<CT>(x0[c]), b = to_c<CT>(y0[c]);
      sum[c] = a + b;
      dif[c] = a - b;
    }
  }
}

// Column sums (for Px) and top-minus-bottom differences (for Py) of three
// rows, once per column.  Out of line for the reason given at gmsd_row.
template <typename CT>
__attribute__((noinline)) void gmsd_cols(const CT* __restrict__ r0, const CT* __restrict__ r1,
                                         const CT* __restrict__ r2, int n, CT* __restrict__ cs,
                                         CT* __restrict__ ds) {
  for (int c = 0; c < n; ++c) {
    cs[c] = (r0[c] + r1[c]) + r2[c];
    ds[c] = r0[c] - r2[c];
  }
}

// d = 1 - q per output column from the column sums / differences of s and e.
//
// The Prewitt filter is linear, so it runs on s = x + y and e = x - y: with
// P = 3 x the Prewitt response, g1 = (Ps + Pe)/2, g2 = (Ps - Pe)/2 and
// G1 - G2 = Pxs Pxe + Pys Pye exactly -- no difference of nearly equal
// magnitudes anywhere, so float32 keeps d to a few ulp for every input type
// but float64, which runs in float64.  G = 9 (gx^2 + gy^2 + eps); T and eps
// carry the same factor 9.
template <typename CT>
__attribute__((noinline)) void gmsd_d(const CT* __restrict__ cs, const CT* __restrict__ ds,
                                      const CT* __restrict__ ce, const CT* __restrict__ de,
                                      int n, CT T9, CT e9, CT* __restrict__ d) {
  for (int c = 0; c < n; ++c) {
    const CT pxs = cs[c] - cs[c + 2];
    const CT pys = (ds[c] + ds[c + 1]) + ds[c + 2];
    const CT pxe = ce[c] - ce[c + 2];
    const CT pye = (de[c] + de[c + 1]) + de[c + 2];
    const CT ax = pxs + pxe, ay = pys + pye, bx = pxs - pxe, by = pys - pye;
    const CT G1 = CT(0.25) * (ax * ax + ay * ay) + e9;
    const CT G2 = CT(0.25) * (bx * bx + by * by) + e9;
    const CT dG = pxs * pxe + pys * pye;
    const CT A = G1 + G2 + CT(2) * std::sqrt(G1 * G2);
    // den is 0 only when G1 = G2 = 0, where dG = 0 too: the floor keeps
    // that 0/0 at 0 without a branch the loop could not vectorise
    const CT den = std::max(A * (G1 + G2 + T9), std::numeric_limits<CT>::min());
    d[c] = (dG * dG) / den;
  }
}

// Sums of d and d^2 over output rows [r0, r1) and Wout output columns of one
// plane (x, y already offset to the tile's first input column, Wd = Wout + 2
// samples wide), each row's sum widened to float64.
template <typename T, typename CT>
void gmsd_band(const T* x, const T* y, int W, int Wd, int Wout, bool down, double T_, double eps,
               int r0, int r1, double* sd, double* sd2) {
  std::vector<CT> rs(static_cast<size_t>(3) * Wd), re(rs.size()), dv(static_cast<size_t>(Wout));
  std::vector<CT> cols(static_cast<size_t>(4) * Wd);
  const CT T9 = static_cast<CT>(9.0 * T_), e9 = static_cast<CT>(9.0 * eps);
  double s = 0.0, s2 = 0.0;
  auto row = [&](std::vector<CT>& v, int r) { return v.data() + static_cast<size_t>(r % 3) * Wd; };
  for (int r = r0; r < r0 + 2; ++r) gmsd_row<T, CT>(x, y, W, Wd, down, r, row(rs, r), row(re, r));
  CT* cs = cols.data();
  CT* ds = cs + Wd;
  CT* ce = ds + Wd;
  CT* de = ce + Wd;
  for (int o = r0; o < r1; ++o) {
    gmsd_row<T, CT>(x, y, W, Wd, down, o + 2, row(rs, o + 2), row(re, o + 2));
    gmsd_cols<CT>(row(rs, o), row(rs, o + 1), row(rs, o + 2), Wd, cs, ds);
    gmsd_cols<CT>(row(re, o), row(re, o + 1), row(re, o + 2), Wd, ce, de);
    gmsd_d<CT>(cs, ds, ce, de, Wout, T9, e9, dv.data());
    row_sums<true>(dv.data(), nullptr, Wout, &s, &s2);
  }
  *sd = s;
  *sd2 = s2;
}

template <typename T>
int gmsd_run(const void* x, const void* y, int N, int C, int H, int W, double T_, double eps,
             bool down, double* out_mean, double* out_std) {
  // tasks: plane x row band x column tile; the per-task sums are combined in
  // task order, so the result does not depend on the thread count
  using CT = typename std::conditional<std::is_same<T, double>::value, double, float>::type;
  const int Hd = down ? H / 2 : H, Wd = down ? W / 2 : W;
  const int Hout = Hd - 2, Wout = Wd - 2;
  if (Hout <= 0 || Wout <= 0) return FA_E_SHAPE;
  const int bands = (Hout + GMSD_BAND - 1) / GMSD_BAND;
  const int tiles = (Wout + GMSD_COLS - 1) / GMSD_COLS;
  const int per_plane = bands * tiles;
  const int64_t planes = static_cast<int64_t>(N) * C;
  std::vector<double> ps(static_cast<size_t>(planes) * per_plane), ps2(ps.size());
  Pool::get().run(planes * per_plane, [&](int64_t t) {
    const int64_t plane = t / per_plane;
    const int rest = static_cast<int>(t - plane * per_plane);
    const int band = rest / tiles, tile = rest - band * tiles;
    const int c0 = tile * GMSD_COLS, cols = std::min(GMSD_COLS, Wout - c0);
    const int64_t in_c0 = down ? 2 * c0 : c0;
    const T* px = static_cast<const T*>(x) + plane * H * W + in_c0;
    const T* py = static_cast<const T*>(y) + plane * H * W + in_c0;
    const int r0 = band * GMSD_BAND;
    gmsd_band<T, CT>(px, py, W, cols + 2, cols, down, T_, eps, r0,
                     std::min(Hout, r0 + GMSD_BAND), &ps[t], &ps2[t]);
  });
  const double n = static_cast<double>(C) * Hout * Wout;
  for (int i = 0; i < N; ++i) {  // fixed order: deterministic
    double s = 0.0, s2 = 0.0;
    for (int64_t k = static_cast<int64_t>(i) * C * per_plane;
         k < static_cast<int64_t>(i + 1) * C * per_plane; ++k) {
      s += ps[k];
      s2 += ps2[k];
    }
    const double md = s / n;
    const double var = s2 / n - md * md;
    out_mean[i] = 1.0 - md;
    out_std[i] = std::sqrt(var > 0.0 ? var : 0.0);
  }
  return FA_OK;
}

}  // namespace facpu

using namespace facpu;

extern "C" {

FA_API int fa_cpu_abi_version(void) { return FA_ABI_VERSION; }

FA_API int fa_cpu_has_avx2(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") ? 1 : 0;
}

FA_API int fa_cpu_set_num_threads(int n) { return Pool::get().set_size(n); }

FA_API int fa_cpu_num_threads(void) { return Pool::get().size(); }

FA_API int fa_cpu_pixel_reduce(const void* a, const void* b, int dtype, int64_t n_images,
                               int64_t n_per_image, int op, double param, double psnr_bias,
                               int per_image, double* out) {
  if (!a || !b || !out) return FA_E_ARG;
  if (op < 0 || op > 3) return FA_E_OP;
  if (dtype < FA_U8 || dtype > FA_F64) return FA_E_DTYPE;
  if (n_images <= 0 || n_per_image <= 0) return FA_E_SHAPE;
  const int64_t chunks = (n_per_image + PIX_CHUNK - 1) / PIX_CHUNK;
  std::vector<double> fsum(static_cast<size_t>(n_images * chunks), 0.0);
  std::vector<uint64_t> isum(fsum.size(), 0);
  std::atomic<bool> exact{false};
  Pool::get().run(n_images * chunks, [&](int64_t t) {
    const int64_t img = t / chunks;
    const int64_t k = t - img * chunks;
    const int64_t off = img * n_per_image + k * PIX_CHUNK;
    const int64_t n = std::min(PIX_CHUNK, n_per_image - k * PIX_CHUNK);
    bool ex = false;
    double f = 0.0;
    switch (dtype) {
      case FA_U8: f = chunk_sum<uint8_t>(op, a, b, off, n, param, &ex, &isum[t]); break;
      case FA_F16: f = chunk_sum<half_t>(op, a, b, off, n, param, &ex, &isum[t]); break;
      case FA_BF16: f = chunk_sum<bf16_t>(op, a, b, off, n, param, &ex, &isum[t]); break;
      case FA_F32: f = chunk_sum<float>(op, a, b, off, n, param, &ex, &isum[t]); break;
      default: f = chunk_sum<double>(op, a, b, off, n, param, &ex, &isum[t]); break;
    }
    fsum[t] = f;
    if (ex) exact.store(true, std::memory_order_relaxed);
  });
  const bool is_exact = exact.load();
  auto image_sum = [&](int64_t img, uint64_t* iacc) {
    double f = 0.0;
    for (int64_t k = 0; k < chunks; ++k) {
      f += fsum[img * chunks + k];
      *iacc += isum[img * chunks + k];
    }
    return f;
  };
  auto finish = [&](double mean) {
    if (psnr_bias == FA_PSNR_NONE) return mean;
    return mean > 0.0 ? psnr_bias - 10.0 * std::log10(mean) : INFINITY;
  };
  if (per_image) {
    for (int64_t img = 0; img < n_images; ++img) {
      uint64_t ia = 0;
      const double f = image_sum(img, &ia);
      const double s = is_exact ? static_cast<double>(ia) : f;
      out[img] = finish(s / static_cast<double>(n_per_image));
    }
  } else {
    uint64_t ia = 0;
    double f = 0.0;
    for (int64_t img = 0; img < n_images; ++img) f += image_sum(img, &ia);
    const double s = is_exact ? static_cast<double>(ia) : f;
    out[0] = finish(s / (static_cast<double>(n_per_image) * static_cast<double>(n_images)));
  }
  return FA_OK;
}

FA_API int fa_cpu_ssim(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                       const float* win, int K, double shift, double C1, double C2,
                       float* map_out, double* out_per_plane) {
  if (!x || !y || !out_per_plane) return FA_E_ARG;
  const int rc = ssim_check(N, C, H, W, win, K);
  if (rc != FA_OK) return rc;
  return ssim_dispatch(x, y, dtype, N, C, H, W, win, K, shift, C1, C2, map_out, out_per_plane,
                       nullptr);
}

FA_API int fa_cpu_ssim_cs(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                          const float* win, int K, double shift, double C1, double C2,
                          double* out_ssim, double* out_cs) {
  if (!x || !y || !out_ssim || !out_cs) return FA_E_ARG;
  int rc = ssim_check(N, C, H, W, win, K);
  if (rc != FA_OK) return rc;
  rc = ssim_dispatch(x, y, dtype, N, C, H, W, win, K, shift, C1, C2, nullptr, out_ssim, out_cs);
  if (rc != FA_OK) return rc;
  const double npix = static_cast<double>(H - K + 1) * (W - K + 1);
  for (int64_t p = 0; p < static_cast<int64_t>(N) * C; ++p) {
    out_ssim[p] /= npix;
    out_cs[p] /= npix;
  }
  return FA_OK;
}

FA_API int fa_cpu_gmsd(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                       double Tc, double eps, int downsample, double* out_mean,
                       double* out_std) {
  if (!x || !y || !out_mean || !out_std) return FA_E_ARG;
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return FA_E_SHAPE;
  const bool down = downsample != 0;
  switch (dtype) {
    case FA_U8: return gmsd_run<uint8_t>(x, y, N, C, H, W, Tc, eps, down, out_mean, out_std);
    case FA_F16: return gmsd_run<half_t>(x, y, N, C, H, W, Tc, eps, down, out_mean, out_std);
    case FA_BF16: return gmsd_run<bf16_t>(x, y, N, C, H, W, Tc, eps, down, out_mean, out_std);
    case FA_F32: return gmsd_run<float>(x, y, N, C, H, W, Tc, eps, down, out_mean, out_std);
    case FA_F64: return gmsd_run<double>(x, y, N, C, H, W, Tc, eps, down, out_mean, out_std);
    default: return FA_E_DTYPE;
  }
}

}  // extern "C"
