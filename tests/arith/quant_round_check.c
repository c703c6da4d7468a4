/* Check of quant_cache's rounding shortcut: with r within 1 ulp of 1/s (v_rcp_f32's bound; r is tried
 * at RN(1/s) and one ulp either side), M = 1.5 * 2^23,
 *   t = fma(x, r, M), e = fma(x, r, -(t - M)),
 * the code clamp(t - M, +-127) equals the IEEE code clamp(rint(fl(x / s)), +-127) whenever
 * |e| < 0.5 - 2^-14 (otherwise the kernel recomputes with IEEE division). x runs over every finite
 * bf16 value (the V path) and 2^20 random fp32 values in (-2^12, 2^12) (the K path's x - mu), s over
 * 2000 scales (log-uniform in [2^-14, 2^6], plus scales that put some x exactly on a tie).
 * Prints the cases checked, the fallbacks taken and the mismatches; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static float clamp127(float c) { return c > 127.f ? 127.f : (c < -127.f ? -127.f : c); }

static uint64_t st = 0x9e3779b97f4a7c15ull;
static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return (uint32_t)(st >> 11); }
static float unif(void) { return (rnd() & 0xffffff) / 16777216.f; }

int main(void) {
  enum { NS = 2000, NX32 = 1 << 20 };
  static float scales[NS];
  static float xs[65536 + NX32];
  int nx = 0;
  for (uint32_t b = 0; b < 65536; ++b) {          /* every finite bf16 */
    const float f = f_of(b << 16);
    if (isfinite(f)) xs[nx++] = f;
  }
  for (int i = 0; i < NX32; ++i) xs[nx++] = (unif() * 2.f - 1.f) * 4096.f;
  for (int i = 0; i < NS; ++i) {
    if (i % 4 == 3) {                               /* x / s exactly k + 0.5 for x = xs[j] */
      const float x = xs[rnd() % 65536];
      const float k = (float)(rnd() % 127) + 0.5f;
      scales[i] = fabsf(x) > 1e-30f ? fabsf(x) / k : 1.f;
      if (!isfinite(scales[i]) || scales[i] < 1e-8f) scales[i] = 1.f;
    } else {
      scales[i] = exp2f(-14.f + 20.f * unif());
    }
  }
  const float M = 12582912.f, thr = 0.5f - 0x1p-14f;
  unsigned long long checked = 0, fallback = 0, bad = 0;
#pragma omp parallel for reduction(+ : checked, fallback, bad) schedule(dynamic)
  for (int i = 0; i < NS; ++i) {
    const float s = scales[i];
    const float r0 = 1.f / s;
    const float rs[3] = {nextafterf(r0, 0.f), r0, nextafterf(r0, INFINITY)};
    for (int k = 0; k < 3; ++k) {
      const float r = rs[k];
      for (int j = 0; j < nx; ++j) {
        const float x = xs[j];
        const float want = clamp127(rintf(x / s));
        const float t = fmaf(x, r, M);
        const float e = fmaf(x, r, -(t - M));
        float got;
        if (fabsf(e) < thr) {
          const float tc = t > M + 127.f ? M + 127.f : (t < M - 127.f ? M - 127.f : t);
          got = tc - M;
        } else {
          ++fallback;
          got = want;                               /* the kernel's exact pass */
        }
        bad += (got != want);
        ++checked;
      }
    }
  }
  printf("checked %llu fallback %llu mismatched %llu\n", checked, fallback, bad);
  return bad != 0;
}
