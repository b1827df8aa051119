/*
 * Exhaustive check of the division-free quotient used by the short-row KV
 * codec kernel (rotalabs-accel_amd/csrc/ra_rowops.hip):
 *
 *   r = RN(1 / s), q0 = RN(x * r), q1 = RN(fma(RN(fma(-q0, s, x)), r, q0))
 *
 * (Markstein's correction). For every 16-bit x and every positive 16-bit
 * scale s >= 1e-8 whose quotient lies in the codec's range |x / s| <= 256,
 * q1 rounded to the 16-bit format must equal RN(x / s) rounded to it (the
 * CPU's true division followed by the tensor dtype's rounding). Also: for
 * every finite non-negative 16-bit x, the same correction gives x / 127 and
 * x / 7 bit-exactly in fp32 (the codec's amax / qmax).
 *
 * Built by tests/test_oracle.py with -ffp-contract=off so that every product
 * and sum is rounded as written; prints the mismatch count and exits non-zero
 * on any mismatch.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16_val(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static float f16_val(uint16_t h) {
  const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024), (int)e - 25);
  return s ? -v : v;
}
static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
/* round to bf16 (RNE) */
static float round_bf16(float f) {
  uint32_t u = bits_of(f);
  u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}
/* round to fp16 (RNE, with subnormals), as an fp32 value */
static float round_f16(float f) {
  if (isnan(f) || isinf(f)) return f;
  const float a = fabsf(f);
  if (a >= 65520.0f) return f > 0 ? INFINITY : -INFINITY;
  int e;
  frexpf(a, &e);
  int q = e - 11;
  if (q < -24) q = -24;
  const float ulp = ldexpf(1.0f, q);
  const float r = rintf(a / ulp) * ulp; /* exact: division by a power of two */
  return f < 0 ? -r : r;
}

int main(void) {
  long long bad = 0, total = 0;
  for (int fmt = 0; fmt < 2; ++fmt) { /* 0: fp16, 1: bf16 */
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, total)
    for (int sb = 1; sb < 0x7F80; ++sb) {
      const float s = fmt ? bf16_val((uint16_t)sb) : f16_val((uint16_t)sb);
      if (!(s >= 1e-8f) || isinf(s) || isnan(s)) continue;
      const float r = 1.0f / s;
      for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
        const float x = fmt ? bf16_val((uint16_t)xb) : f16_val((uint16_t)xb);
        if (!isfinite(x)) continue;
        const float ref = x / s;
        if (!(fabsf(ref) <= 256.0f)) continue;
        const float q0 = x * r;
        const float q1 = fmaf(fmaf(-q0, s, x), r, q0);
        const float a = fmt ? round_bf16(q1) : round_f16(q1);
        const float b = fmt ? round_bf16(ref) : round_f16(ref);
        ++total;
        if (bits_of(a) != bits_of(b) && !(a == 0 && b == 0)) ++bad;
      }
    }
  }
  /* amax / qmax */
  const float cs[2] = {127.0f, 7.0f};
  for (int fmt = 0; fmt < 2; ++fmt)
    for (int ci = 0; ci < 2; ++ci) {
      const float c = cs[ci], r = 1.0f / c;
      for (uint32_t xb = 0; xb < 0x8000u; ++xb) {
        const float x = fmt ? bf16_val((uint16_t)xb) : f16_val((uint16_t)xb);
        if (!isfinite(x)) continue;
        const float q0 = x * r;
        const float q1 = fmaf(fmaf(-q0, c, x), r, q0);
        ++total;
        if (bits_of(q1) != bits_of(x / c)) ++bad;
      }
    }
  printf("%lld cases, %lld mismatches\n", total, bad);
  return bad != 0;
}
