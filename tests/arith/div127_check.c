/* Exhaustive check of the attention kernel's P-tile scale: for every float x in [2^-126, 1],
 * fma(fma(-q, 127, x), R, q) with q = fl(x * R), R = fl(1/127), equals the IEEE quotient fl(x / 127).
 * Prints the number of values checked and mismatched; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
  const float R = 1.f / 127.f;
  const uint32_t lo = 0x00800000u, hi = 0x3f800000u; /* 2^-126 .. 1.0 */
  unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long i = lo; i <= (long long)hi; ++i) {
    const uint32_t u = (uint32_t)i;
    float x;
    memcpy(&x, &u, 4);
    const float q = x * R;
    const float r = fmaf(fmaf(-q, 127.f, x), R, q);
    const float ref = x / 127.f;
    bad += (r != ref);
  }
  printf("checked %llu mismatched %llu\n", (unsigned long long)(hi - lo + 1), bad);
  return bad != 0;
}
