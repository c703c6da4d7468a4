/* Check of code_magic, the division-free code of the cache write and the q quantization: with
 * y = fl(1 / s) (IEEE division) and M = 1.5 * 2^23,
 *   q = clamp(fl(x * y), +-254), f = fma(fma(-q, s, x), y, q), t = clamp(fl(f + M), M +- 127),
 * t - M must equal the IEEE code clamp(rint(fl(x / s)), +-127) for every x and s. x runs over every
 * bf16 value but the NaNs (infinities included: the V path), 2^20 random fp32 values in (-2^12, 2^12)
 * (the K path's x - mu) and, per scale, fp32 values on and within 4 ulps of 256 half-integer
 * quotients; s over 2400 scales: log-uniform in [2^-14, 2^6], a bf16 absolute maximum / 127 (the
 * calibration's form, which puts many bf16 x exactly on ties) and scales that put a chosen x exactly
 * on a tie. Prints the cases checked and the mismatches; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float clamp(float c, float lo, float hi) { return c > hi ? hi : (c < lo ? lo : c); }

static uint64_t st = 0x2545f4914f6cdd1dull;
static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return (uint32_t)(st >> 11); }
static float unif(void) { return (rnd() & 0xffffff) / 16777216.f; }

static float code_ieee(float x, float s) { return clamp(rintf(x / s), -127.f, 127.f); }
static float code_magic(float x, float s, float y) {
  const float M = 12582912.f;
  const float q = clamp(x * y, -254.f, 254.f);
  const float f = fmaf(fmaf(-q, s, x), y, q);
  return clamp(f + M, M - 127.f, M + 127.f) - M;
}

int main(void) {
  enum { NS = 2400, NX32 = 1 << 20, NTIE = 256 };
  static float scales[NS];
  static float xs[65536 + NX32];
  int nx = 0;
  for (uint32_t b = 0; b < 65536; ++b) {          /* every bf16 but NaN */
    const float f = f_of(b << 16);
    if (!isnan(f)) xs[nx++] = f;
  }
  for (int i = 0; i < NX32; ++i) xs[nx++] = (unif() * 2.f - 1.f) * 4096.f;
  for (int i = 0; i < NS; ++i) {
    if (i % 3 == 1) {                               /* bf16 absolute maximum / 127 */
      scales[i] = f_of(((rnd() % 0x1f00u) + 0x3100u) << 16) / 127.f;
    } else if (i % 3 == 2) {                        /* x / s exactly k + 0.5 for a chosen bf16 x */
      const float x = fabsf(xs[rnd() % 65536]);
      const float k = (float)(rnd() % 127) + 0.5f;
      scales[i] = (isfinite(x) && x > 1e-30f) ? x / k : 1.f;
      if (!isfinite(scales[i]) || scales[i] < 1e-8f || scales[i] > 1e8f) scales[i] = 1.f;
    } else {
      scales[i] = exp2f(-14.f + 20.f * unif());
    }
  }
  unsigned long long checked = 0, bad = 0;
#pragma omp parallel for reduction(+ : checked, bad) schedule(dynamic)
  for (int i = 0; i < NS; ++i) {
    const float s = scales[i];
    const float y = 1.f / s;
    for (int j = 0; j < nx; ++j) {
      bad += code_magic(xs[j], s, y) != code_ieee(xs[j], s);
      ++checked;
    }
    uint64_t ls = 0x9e3779b97f4a7c15ull ^ (uint64_t)i;
    for (int t = 0; t < NTIE; ++t) {                /* on and next to half-integer quotients */
      ls ^= ls << 13; ls ^= ls >> 7; ls ^= ls << 17;
      const float k = (float)((int)(ls % 255u) - 127) + 0.5f;
      const uint32_t c = u_of(k * s);
      for (int d = -4; d <= 4; ++d) {
        const float x = f_of(c + (uint32_t)d);
        bad += code_magic(x, s, y) != code_ieee(x, s);
        ++checked;
      }
    }
  }
  printf("checked %llu mismatched %llu\n", checked, bad);
  return bad != 0;
}
