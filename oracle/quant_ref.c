/* TEST INFRASTRUCTURE ONLY -- an independent C restatement of the element formulas of the static
 * INT8 KV-cache path, used by tests/ to cross-check the PyTorch oracle (oracle/kvq_oracle.py) and
 * the HIP kernels. Never linked into the product.
 *
 *   code    = sat127(rintf(fl32(x / s)))          kvq/quant.py:50-51 (IEEE division, ties to even)
 *   dequant = bf16_rne(fl32((float)code * s))      kvq/quant.py:54-55 with dtype=bfloat16
 *   q codes = code(fl32(f32(q) * s_k), max(amax / 127, 1e-8))   tests/test_cuda_kernels.py:52-54
 * Built with -ffp-contract=off so that no product or difference is fused.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float sat127(float n) { return n < -127.f ? -127.f : (n > 127.f ? 127.f : n); }

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* out[i] = sat127(rintf(x[i] / s[i % period])) */
void oracle_codes(const float* x, const float* s, int64_t n, int64_t period, int8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (int8_t)sat127(rintf(x[i] / s[i % period]));
}

/* rows of bf16 [rows, H*D]: out = code(f32(x) - mu, s); mu may be NULL; s has H*D entries
 * (per channel) or H entries (per head, s_cols == 1). */
void oracle_quant_rows(const uint16_t* x, const float* mu, const float* s, int64_t rows, int64_t H, int64_t D,
                       int64_t s_cols, int8_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t d = 0; d < D; ++d) {
        const int64_t c = h * D + d;
        float v = bf16_to_f32(x[r * H * D + c]);
        if (mu) v = v - mu[c];
        const float sc = s_cols > 1 ? s[c] : s[h];
        out[r * H * D + c] = (int8_t)sat127(rintf(v / sc));
      }
}

/* bf16 bits of (float)code * s */
void oracle_dequant(const int8_t* q, const float* s, int64_t rows, int64_t H, int64_t D, int64_t s_cols,
                    uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t d = 0; d < D; ++d) {
        const int64_t c = h * D + d;
        const float sc = s_cols > 1 ? s[c] : s[h];
        out[r * H * D + c] = f32_to_bf16((float)q[r * H * D + c] * sc);
      }
}

/* q codes of one row per (token, q head): q bf16 [rows, D] with kv head kvh(row) = (row % Hq) / G,
 * ks [Hkv, D] (folded when ks_cols > 1), one scale per `group` channels. */
void oracle_quant_q(const uint16_t* q, const float* ks, int64_t rows, int64_t Hq, int64_t G, int64_t D,
                    int64_t ks_cols, int64_t group, int8_t* codes, float* scales) {
  float x[256];
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t kvh = (r % Hq) / G;
    for (int64_t d = 0; d < D; ++d) {
      x[d] = bf16_to_f32(q[r * D + d]);
      if (ks_cols > 1) x[d] = x[d] * ks[kvh * D + d];
    }
    for (int64_t g0 = 0; g0 < D; g0 += group) {
      float amax = 0.f;
      for (int64_t d = g0; d < g0 + group; ++d) amax = fabsf(x[d]) > amax ? fabsf(x[d]) : amax;
      float s = amax / 127.f;
      if (s < 1e-8f) s = 1e-8f;
      scales[r * (D / group) + g0 / group] = s;
      for (int64_t d = g0; d < g0 + group; ++d) codes[r * D + d] = (int8_t)sat127(rintf(x[d] / s));
    }
  }
}
