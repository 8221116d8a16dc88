// Division of 32-bit row indices by a launch-invariant divisor with one
// multiply-high, an add and a shift (Granlund & Montgomery, "Division by
// Invariant Integers using Multiplication", PLDI 1994, round-up method):
//
//   l = ceil(log2 d),  m = floor(2^32 (2^l - d) / d) + 1,
//   n / d = (mulhi(n, m) + n) >> l      for 0 <= n < 2^31, 1 <= d < 2^31.
//
// mulhi(n, m) <= n, so the add cannot carry out of 32 bits for n < 2^31.
// Plain C++ so the host test (tests/test_fastdiv.py) compiles this same text.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define XGEN_HD __host__ __device__
#else
#define XGEN_HD
#endif

namespace xgen {

struct FastDiv {
  uint32_t d;  // divisor
  uint32_t m;  // magic multiplier
  uint32_t l;  // shift
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  f.l = l;
  f.m = (uint32_t)((((1ull << 32) * ((1ull << l) - d)) / d) + 1);
  return f;
}

XGEN_HD inline uint32_t fast_div(uint32_t n, const FastDiv &f) {
  const uint32_t hi = (uint32_t)(((uint64_t)n * f.m) >> 32);
  return (hi + n) >> f.l;
}

}  // namespace xgen
