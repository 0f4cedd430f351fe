// Host check of fa_fastdiv.h (compiled and run by tests/test_fastdiv.py):
// every n < 2^18 for every divisor d < 2^12, plus n near 2^31 and the
// divisors near 2^31, against the hardware division.
#include <stdio.h>
#include "fa_fastdiv.h"

int main() {
  long long bad = 0, checked = 0;
  for (uint32_t d = 1; d < 4096; ++d) {
    const fa::FastDiv f = fa::make_fastdiv(d);
    for (uint32_t n = 0; n < (1u << 18); ++n, ++checked)
      if (fa::fdiv(n, f) != n / d || fa::fmod(n, f) != n % d) ++bad;
    for (uint32_t n = 0x7fffffffu - 5000; n <= 0x7fffffffu - 1; ++n, ++checked)
      if (fa::fdiv(n, f) != n / d) ++bad;
  }
  for (uint32_t d = 0x7fffffffu - 100; d < 0x7fffffffu; ++d) {
    const fa::FastDiv f = fa::make_fastdiv(d);
    for (uint32_t n = 0x7fffffffu - 1000; n < 0x7fffffffu; ++n, ++checked)
      if (fa::fdiv(n, f) != n / d) ++bad;
    for (uint32_t n = 0; n < 1000; ++n, ++checked)
      if (fa::fdiv(n, f) != n / d) ++bad;
  }
  printf("checked %lld, wrong %lld\n", checked, bad);
  return bad != 0;
}
