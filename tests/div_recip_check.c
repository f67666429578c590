/* CPU check of the softmax's quotient by a shared divisor: for b in [1, 2^16]
 * and y = 1.0f / b, q = a*y, r = fma(-b, q, a), fma(r, y, q) equals the IEEE
 * quotient a / b. Every a in [2^-86, 1] (the nonzero probabilities' numerators
 * the kernel sends this way) is tried for each divisor given on the command
 * line as a bit pattern; prints the number of mismatches. Build with FMA
 * hardware for speed (-O2 -mfma); fmaf is exact either way. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char **argv) {
  const uint32_t lo = 0x14800000u, hi = 0x3f800000u; /* 2^-86, 1 */
  long long total = 0;
  for (int j = 1; j < argc; j++) {
    const float b = u2f((uint32_t)strtoul(argv[j], NULL, 0));
    const float y = 1.0f / b;
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t u = lo; u <= (int64_t)hi; u++) {
      const float a = u2f((uint32_t)u);
      const float q = a * y;
      const float r = fmaf(-b, q, a);
      bad += f2u(fmaf(r, y, q)) != f2u(a / b);
    }
    if (bad) printf("b=%.9g: %lld\n", b, bad);
    total += bad;
  }
  printf("%lld\n", total);
  return 0;
}
