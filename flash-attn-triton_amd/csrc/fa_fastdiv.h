// Division by a runtime divisor that is the same for a whole kernel (head
// counts, blocks per group, GQA group size), as a multiply-high and a shift.
//
// For 1 <= d < 2^31 let l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1
// (computed once, with one 64-bit division); then for 0 <= n < 2^31
//   n / d = (umulhi(n, m) + n) >> l
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4, with the sum kept below 2^32 by the
// bound on n).  Plain C++ so that host tests compile the same code; on the
// GPU a uniform operand makes it two scalar instructions (s_mul_hi_u32,
// s_add, s_lshr) instead of a division routine.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FA_HD __host__ __device__
#else
#define FA_HD
#endif

namespace fa {

struct FastDiv {
  uint32_t d, m, l;
};

FA_HD inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while (l < 31 && (uint32_t(1) << l) < d) ++l;
  const uint64_t m = (uint64_t(1) << 32) * ((uint64_t(1) << l) - d) / d + 1;
  return FastDiv{d, (uint32_t)m, l};
}

// n / f.d for 0 <= n < 2^31.
FA_HD inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
  const uint32_t t = (uint32_t)(((uint64_t)n * f.m) >> 32);
  return (t + n) >> f.l;
}

// n % f.d for 0 <= n < 2^31.
FA_HD inline uint32_t fmod(uint32_t n, const FastDiv& f) { return n - fdiv(n, f) * f.d; }

}  // namespace fa
