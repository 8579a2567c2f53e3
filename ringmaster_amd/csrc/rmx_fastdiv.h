// Division of non-negative 32-bit indices by a runtime divisor with one
// multiply-high (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant with a 33-bit multiplier):
//   s = ceil(log2 d), m = floor(2^(32+s) / d) + 1 - 2^32,
//   n / d = (umulhi(n, m) + n) >> s     exact for 0 <= n < 2^31, 1 <= d < 2^31.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rmx {

struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)(((1ull << (32 + s)) / d) + 1 - (1ull << 32));
  return f;
}

__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
#ifdef __HIP_DEVICE_COMPILE__
  const uint32_t hi = __umulhi(n, f.m);
#else
  const uint32_t hi = (uint32_t)(((uint64_t)n * f.m) >> 32);
#endif
  return (hi + n) >> f.s;
}

}  // namespace rmx
