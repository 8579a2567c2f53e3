// Host check of rmx_fastdiv.h: fdiv(n, make_fastdiv(d)) == n / d for edge and
// random (n, d), 0 <= n < 2^31, 1 <= d < 2^31. Exit status 0 when all agree.
#include <cstdio>
#include <random>

#include "rmx_fastdiv.h"

int main() {
  std::mt19937_64 gen(7);
  long bad = 0, total = 0;
  const uint32_t ds[] = {1, 2, 3, 5, 7, 8, 16, 31, 256, 1000, 16384, 16385, 65535, 1u << 20,
                         3u * (1u << 20) + 7, 1u << 30, (1u << 31) - 1};
  auto check = [&](uint32_t n, uint32_t d, const rmx::FastDiv& f) {
    ++total;
    if (rmx::fdiv(n, f) != n / d) {
      if (bad < 10) std::printf("mismatch n=%u d=%u\n", n, d);
      ++bad;
    }
  };
  for (uint32_t d : ds) {
    const rmx::FastDiv f = rmx::make_fastdiv(d);
    const uint32_t top = (1u << 31) - 1;
    for (uint32_t n : {0u, 1u, d - 1, d, d + 1, top, top - 1, top / d * d, top / d * d - 1})
      if (n <= top) check(n, d, f);
    for (int i = 0; i < 100000; ++i) check((uint32_t)(gen() % (1u << 31)), d, f);
  }
  for (int i = 0; i < 500000; ++i) {
    const uint32_t d = 1 + (uint32_t)(gen() % ((1u << 31) - 1));
    check((uint32_t)(gen() % (1u << 31)), d, rmx::make_fastdiv(d));
  }
  std::printf("fastdiv: %ld checked, %ld mismatches\n", total, bad);
  return bad != 0;
}
