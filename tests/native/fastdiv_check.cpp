// Exhaustive / edge checks of voiceagent_amd/csrc/fastdiv.h against the
// hardware integer division: every divisor 1..4096 over n in [0, 2^17) and
// at the top of the range, plus large, prime and power-of-two divisors at
// the multiples of d around 2^31.
#include <cstdio>
#include <cstdint>
#include <vector>

#include "../../voiceagent_amd/csrc/fastdiv.h"

static int check(uint32_t d, uint32_t n) {
  const va::FastDiv f = va::make_fastdiv(d);
  if (va::fast_div(n, f) != n / d || va::fast_mod(n, f) != n % d) {
    std::printf("FAIL d=%u n=%u got %u want %u\n", d, n, va::fast_div(n, f), n / d);
    return 1;
  }
  return 0;
}

int main() {
  const uint32_t top = 0x7fffffffu;
  for (uint32_t d = 1; d <= 4096; ++d) {
    for (uint32_t n = 0; n < (1u << 17); ++n)
      if (check(d, n)) return 1;
    for (uint32_t n = top - 70000; n < top; ++n)
      if (check(d, n)) return 1;
    if (check(d, top)) return 1;
  }
  std::vector<uint32_t> big = {4097, 65535, 65536, 65537, 1000003, 16777215, 16777216,
                               16777217, 1u << 30, (1u << 30) + 1, 2147483629u, top, 1u << 31};
  for (uint32_t d : big) {
    for (uint64_t k = 0; k * d <= top; k += (k < 1000 ? 1 : (top / d) / 1000 + 1))
      for (int64_t e = -2; e <= 2; ++e) {
        const int64_t n = (int64_t)(k * d) + e;
        if (n >= 0 && n <= top && check(d, (uint32_t)n)) return 1;
      }
    for (uint32_t n = top - 5000; n < top; ++n)
      if (check(d, n)) return 1;
    if (check(d, top)) return 1;
  }
  std::printf("ok\n");
  return 0;
}
