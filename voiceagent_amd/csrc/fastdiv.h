// Division by a runtime divisor fixed for a launch, as one 32 x 32 -> 64-bit
// multiply and a shift (Granlund and Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994), for dividends in [0, 2^31).
//
// For a divisor d >= 1 let l = ceil(log2 d) and m = ceil(2^(31 + l) / d).
// Then m < 2^32, and for every n in [0, 2^31)
//     floor(n / d) = floor(n m / 2^(31 + l)):
// with m = 2^(31 + l) / d + e, 0 <= e < 1, the product is n / d + n e / 2^(31 + l),
// and n e / 2^(31 + l) < 2^-l <= 1 / d, which cannot carry n / d past the next
// integer (its fractional part is at most (d - 1) / d).
//
// Plain C++ with no GPU dependency, so the host side is testable on its own.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define VA_HD __host__ __device__
#else
#define VA_HD
#endif

namespace va {

struct FastDiv {
  uint32_t mul;    // ceil(2^shift / d)
  uint32_t shift;  // 31 + ceil(log2 d)
  uint32_t d;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d < 1 ? 1 : d;
  uint32_t l = 0;
  while (((uint64_t)1 << l) < f.d) ++l;
  f.shift = 31 + l;
  f.mul = (uint32_t)((((uint64_t)1 << f.shift) + f.d - 1) / f.d);
  return f;
}

// floor(n / f.d) for n in [0, 2^31).
VA_HD inline uint32_t fast_div(uint32_t n, const FastDiv& f) {
  return (uint32_t)(((uint64_t)n * f.mul) >> f.shift);
}

// n mod f.d for n in [0, 2^31).
VA_HD inline uint32_t fast_mod(uint32_t n, const FastDiv& f) { return n - fast_div(n, f) * f.d; }

}  // namespace va
