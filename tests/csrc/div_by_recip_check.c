/* Checks the division used by the router's softmax: with y = RN(1/b),
 *   q0 = RN(a*y), rem = fma(-q0, b, a), q = RN(fma(rem, y, q0))
 * must equal the IEEE quotient RN(a/b).  Every significand of a is tried at
 * the given exponents, against divisors b in [1, 2048) drawn from a fixed
 * generator plus the significands next to 1 and 2.  Prints the number of
 * mismatches (0 expected).  Usage: div_by_recip_check NB EXP...           */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  const int nb = atoi(argv[1]);
  long bad = 0, total = 0;
  uint32_t state = 0x9e3779b9u;
  for (int j = 0; j < nb; ++j) {
    state ^= state << 13; state ^= state >> 17; state ^= state << 5;
    uint32_t sig = state & 0x7fffffu;
    if (j < 4) sig = 0x7fffffu - (uint32_t)j;     /* just below 2 */
    else if (j < 8) sig = (uint32_t)(j - 4);      /* 1 and just above */
    const float b = ldexpf(from_bits(0x3f800000u | sig), j % 11);
    volatile float one = 1.0f;
    const float y = one / b;
    for (int ai = 2; ai < argc; ++ai) {
      const int ex = atoi(argv[ai]);
      for (uint32_t m = 0; m < (1u << 23); ++m) {
        const float a = ldexpf(from_bits(0x3f800000u | m), ex);
        const float q0 = a * y;
        const float rem = fmaf(-q0, b, a);
        const float q = fmaf(rem, y, q0);
        const float ref = a / b;
        ++total;
        bad += to_bits(q) != to_bits(ref);
      }
    }
  }
  printf("%ld %ld\n", total, bad);
  return 0;
}
