/* Exhaustive check of the INT8 Q quantizer's division (quant_div in
 * flash-attn-triton_amd/csrc/fa_int8.h): for every finite fp16 amax and
 * every fp16 x with |x| <= amax, the quotient from the correctly rounded
 * reciprocal with one Markstein correction,
 *   inv = 1 / s,  q0 = x * inv,  r = fma(-q0, s, x),  q = fma(r, inv, q0),
 * equals the IEEE fp32 division x / s, s = fp32(max(amax, 1)) / 127.
 * Every amax below 1 gives s = 1 / 127, covered once.  Prints the pair count
 * and the number of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t bits;
  if (e == 0) {
    float f = ldexpf((float)m, -24);
    memcpy(&bits, &f, 4);
    bits |= sign;
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

int main(void) {
  long long pairs = 0, bad = 0;
  for (uint32_t ha = 0; ha < 0x7c00u; ++ha) {
    const float amax = half_to_float((uint16_t)ha);
    if (amax < 1.0f && ha != 0x3bffu) continue;
    const float s = fmaxf(amax, 1.0f) / 127.0f;
    const float inv = 1.0f / s;
    const float lim = fmaxf(amax, 1.0f) > amax && amax < 1.0f ? 1.0f : amax;
    for (uint32_t hx = 0; hx < 0x10000u; ++hx) {
      if ((hx & 0x7c00u) == 0x7c00u) continue;
      const float x = half_to_float((uint16_t)hx);
      if (fabsf(x) > lim) continue;
      const float q0 = x * inv;
      const float r = fmaf(-q0, s, x);
      const float q = fmaf(r, inv, q0);
      ++pairs;
      if (q != x / s) ++bad;
    }
  }
  printf("%lld %lld\n", pairs, bad);
  return 0;
}
