// Device helpers shared by the linear-scan kernels (scan.hip, scan_chunked.hip).
#pragma once
#include <type_traits>

#include "rmx_common.h"

namespace rmx {

// V consecutive fp32 channels (V = 1, 2, 4) as one load / store. Every
// channel row is read once per pass, so the loads are non-temporal too.
template <int V>
__device__ __forceinline__ void ldv(const float* p, float* o) {
  if constexpr (V == 4) {
    const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
#pragma unroll
    for (int v = 0; v < 4; ++v) o[v] = x[v];
  } else if constexpr (V == 2) {
    const f32x2 x = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(p));
    o[0] = x[0];
    o[1] = x[1];
  } else {
    o[0] = __builtin_nontemporal_load(p);
  }
}
// Stores are non-temporal: the scan outputs stream past the caches (h is read
// back only by the backward, long after).
template <int V>
__device__ __forceinline__ void stv(float* p, const float* o) {
  if constexpr (V == 4) {
    __builtin_nontemporal_store(f32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<f32x4*>(p));
  } else if constexpr (V == 2) {
    __builtin_nontemporal_store(f32x2{o[0], o[1]}, reinterpret_cast<f32x2*>(p));
  } else {
    __builtin_nontemporal_store(o[0], p);
  }
}

// Sum over the 64 lanes of a wave of 16 per-lane values (one per step): a
// transposing butterfly in which, at the stage with mask M, each lane keeps the
// half of its partial sums selected by lane bit M and adds the partner's copy
// of that half (17 exchanges for 16 steps). Returns the wave sum of step
// u = 8 b5 + 4 b4 + 2 b3 + b2 of the lane (b = lane bits, so the lanes with
// b1 = b0 = 0 hold all 16 steps between them) and sets `u`.
__device__ __forceinline__ float wave_sum16(float (&part)[16], int lane, int& u) {
  auto stage = [&](auto mask, auto halfc) {
    constexpr int M = decltype(mask)::value, H = decltype(halfc)::value;
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float keep = hi ? part[H + i] : part[i];
      const float send = hi ? part[i] : part[H + i];
      part[i] = keep + __shfl_xor(send, M, 64);
    }
  };
  stage(std::integral_constant<int, 32>{}, std::integral_constant<int, 8>{});
  stage(std::integral_constant<int, 16>{}, std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 8>{}, std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 4>{}, std::integral_constant<int, 1>{});
  float x = part[0];
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 1, 64);
  u = ((lane >> 2) & 1) | (((lane >> 3) & 1) << 1) | (((lane >> 4) & 1) << 2) |
      (((lane >> 5) & 1) << 3);
  return x;
}

}  // namespace rmx
