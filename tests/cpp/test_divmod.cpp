// Checks sa::FastDiv (csrc/kernels/divmod.h, host path) against exact
// integer division: every divisor up to 4096, then edge divisors near powers
// of two and the 2^31 limit, each against edge dividends and random ones.
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "divmod.h"

int main() {
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (int s = 12; s <= 31; ++s) {
    const uint32_t p = 1u << s;
    for (int k = -3; k <= 3; ++k) {
      const int64_t d = (int64_t)p + k;
      if (d >= 1 && d <= (int64_t(1) << 31)) divisors.push_back((uint32_t)d);
    }
  }
  divisors.push_back(128256);
  divisors.push_back(1048576);
  std::mt19937 rng(1234);
  long checks = 0;
  for (uint32_t d : divisors) {
    sa::FastDiv f(d);
    std::vector<uint32_t> ns = {0u, 1u, d - 1, d, d + 1, 0x7fffffffu, 0x80000000u, 0xfffffffeu, 0xffffffffu};
    for (int i = 0; i < 2000; ++i) ns.push_back(rng());
    for (uint32_t k = 1; k < 5; ++k) ns.push_back((uint32_t)((uint64_t)d * k - 1));
    for (uint32_t n : ns) {
      uint32_t q, r;
      f.divmod(n, q, r);
      if (q != n / d || r != n % d) {
        std::printf("FAIL d=%u n=%u got q=%u r=%u\n", d, n, q, r);
        return 1;
      }
      ++checks;
    }
  }
  std::printf("OK %ld checks\n", checks);
  return 0;
}
