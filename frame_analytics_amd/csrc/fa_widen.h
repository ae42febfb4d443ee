// Exact float -> double widening in integer arithmetic, for the strip
// engine's float64 window weights.  Host-callable too: tests/test_widen.py
// compiles it with g++ and compares it with the conversion for every float
// bit pattern.
#pragma once

#include <cstdint>

namespace fa {

// float -> double of a workgroup-uniform value in integer arithmetic, so the
// result stays in scalar registers (the vector conversion would put it in
// vector ones).  Exact like the conversion: the exponent is rebiased
// (127 -> 1023), the mantissa moves to the top of the 52-bit field, a
// subnormal is normalised, and infinities / NaNs keep their payload.
__host__ __device__ inline double widen_uniform(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint64_t sign = static_cast<uint64_t>(u >> 31) << 63;
  const uint32_t e = (u >> 23) & 0xffu;
  const uint32_t m = u & 0x7fffffu;
  uint64_t bits;
  if (e == 0xffu) {  // a NaN comes out quiet, as from the conversion
    bits = sign | (0x7ffull << 52) | (static_cast<uint64_t>(m) << 29) | (m ? 1ull << 51 : 0);
  } else if (e != 0) {
    bits = sign | (static_cast<uint64_t>(e + 896u) << 52) | (static_cast<uint64_t>(m) << 29);
  } else if (m == 0) {
    bits = sign;
  } else {
    const int sh = __builtin_clz(m) - 8;  // moves the leading 1 to bit 23
    bits = sign | (static_cast<uint64_t>(897 - sh) << 52) |
           (static_cast<uint64_t>((m << sh) & 0x7fffffu) << 29);
  }
  return __builtin_bit_cast(double, bits);
}

}  // namespace fa
