// Read-bandwidth ceiling, for bench.py only (not part of the metric ABI).
//
// The fastest pure streaming read of N bytes this GPU sustains: each lane
// keeps U 16-byte loads per buffer in flight and folds them with one XOR per
// dword, so nothing but the loads costs time.  bench.py sweeps U, the block
// size and the blocks per CU and reports the best, as the attainable figure
// beside the 8 TB/s data-sheet peak.
//
// Two layouts, both reading exactly `bytes` per launch:
//   pair: two buffers of bytes/2 walked in lockstep by one grid-wide stride
//         (the access pattern of the PSNR/MSE sweep over a and b)
//   flat: one buffer of `bytes`
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// Loads at v + u * stride are issued only while v + (U - 1) * stride < nvec,
// and the tail loop only while v < nvec: every access stays inside the buffers.
template <int U>
__global__ __launch_bounds__(1024) void read_pair(const u32x4* __restrict__ a,
                                                  const u32x4* __restrict__ b, int64_t nvec,
                                                  uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; v + (U - 1) * stride < nvec; v += U * stride) {
    u32x4 xa[U], xb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xa[u] = __builtin_nontemporal_load(a + v + u * stride);
      xb[u] = __builtin_nontemporal_load(b + v + u * stride);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= fold(xa[u]) ^ fold(xb[u]);
  }
  for (; v < nvec; v += stride) acc ^= fold(a[v]) ^ fold(b[v]);
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads; a vector store
}

template <int U>
__global__ __launch_bounds__(1024) void read_flat(const u32x4* __restrict__ a, int64_t nvec,
                                                  uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; v + (U - 1) * stride < nvec; v += U * stride) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(a + v + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= fold(x[u]);
  }
  for (; v < nvec; v += stride) acc ^= fold(a[v]);
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

template <int U>
void launch(const void* a, const void* b, int64_t nvec, int blocks, int block, uint32_t* sink,
            hipStream_t st) {
  const auto* pa = static_cast<const u32x4*>(a);
  if (b)
    hipLaunchKernelGGL(read_pair<U>, dim3(blocks), dim3(block), 0, st, pa,
                       static_cast<const u32x4*>(b), nvec, sink);
  else
    hipLaunchKernelGGL(read_flat<U>, dim3(blocks), dim3(block), 0, st, pa, nvec, sink);
}

}  // namespace

// bytes: bytes of each buffer (a multiple of 16; a and b 16-byte aligned);
// b null reads `a` alone.  unroll in {1, 2, 4, 8}; block a multiple of 64
// up to 1024.  Returns 0, 1 for a bad argument, or -hipError_t.
extern "C" __attribute__((visibility("default"))) int fa_readbw_launch(
    const void* a, const void* b, int64_t bytes, int unroll, int blocks, int block,
    uint32_t* sink, void* stream) {
  if (!a || !sink || bytes <= 0 || bytes % 16 != 0 || blocks <= 0 || block <= 0 ||
      block > 1024 || block % 64 != 0)
    return 1;
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) return 1;
  const int64_t nvec = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (unroll) {
    case 1: launch<1>(a, b, nvec, blocks, block, sink, st); break;
    case 2: launch<2>(a, b, nvec, blocks, block, sink, st); break;
    case 4: launch<4>(a, b, nvec, blocks, block, sink, st); break;
    case 8: launch<8>(a, b, nvec, blocks, block, sink, st); break;
    default: return 1;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -static_cast<int>(e);
}
