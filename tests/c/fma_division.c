/* Checks the FMA-refined quotient the quantize kernels use instead of an fp32
 * division per element:
 *   r = RN(1 / s);  q = RN(x * r);  e' = RN(q * s - x) (one FMA, exact);
 *   q' = RN(q - e' * r) (one FMA). With the residual negated, a zero x keeps its
 *   sign: q = +-0, e' = +0 and q' = -0 + q (x - q * s would give +0 + -0 = +0).
 * Claim: q' == RN(x / s) bit for bit whenever |x| >= 2^-100 and x / s is a
 * normal float (Markstein's correction step: r is the correctly rounded
 * reciprocal, q is within one ulp of x / s, and the residual e is exact
 * because it stays in the normal range); for smaller |x| the residual can
 * underflow, and q' is then below 2^-40 in magnitude with the sign of x, as
 * x / s is (both round to the same signed zero in int8 and FP8, whose
 * smallest nonzero magnitude is 2^-9). For every x, rint(q') == rint(x / s),
 * the integer the int8 path keeps.
 * Inputs: every finite bf16 value and pseudo-random fp32 bit patterns as x;
 * scales s = RN(amax / 127) and RN(amax / 448) over amax from every bf16
 * binade and random magnitudes, plus all-ones and one mantissas in each
 * binade. Prints "checked <n> mismatches <m>". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* c = s, or 0 for an infinite s (the kernels' correction multiplier) */
static float div_fma(float x, float c, float r) {
  const float q = x * r;
  const float e = fmaf(q, c, -x);
  return fmaf(-e, r, q);
}

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t next_u32(void) {
  rng_state ^= rng_state << 13; rng_state ^= rng_state >> 7; rng_state ^= rng_state << 17;
  return (uint32_t)(rng_state >> 16);
}

static long long checked = 0, bad = 0;

static void check(float x, float s) {
  const float want = x / s;
  const float got = div_fma(x, isinf(s) ? 0.0f : s, 1.0f / s);
  if (!isfinite(want) || fabsf(want) > 0x1p100f) return;  /* quantized rows keep |x / s| <= 448 */
  ++checked;
  if (signbit(got) != signbit(x)) ++bad;  /* x / s has the sign of x, zeros included (-0 -> 0x80) */
  if (fabsf(x) >= 0x1p-100f && fabsf(want) >= 0x1p-126f) {
    if (u_of(got) != u_of(want)) ++bad;
  } else if (fabsf(x) < 0x1p-100f) {
    if (!(fabsf(got) <= 0x1p-40f && fabsf(want) <= 0x1p-40f && signbit(got) == signbit(x))) ++bad;
  }
  if (fabsf(want) <= 256.0f && rintf(got) != rintf(want)) ++bad;
}

int main(void) {
  float scales[8192];
  int ns = 0;
  scales[ns++] = 1.0f; scales[ns++] = 0x1p-20f; scales[ns++] = INFINITY; scales[ns++] = 1e-12f / 127.0f; scales[ns++] = 1e-12f / 448.0f;
  for (int e = -40; e < 40; e += 3) {
    scales[ns++] = ldexpf(1.9999999f, e);
    scales[ns++] = ldexpf(1.0000001f, e);
  }
  for (uint32_t b = 0; b < 0x7f80u && ns < 8000; b += 37) {  /* positive finite bf16 amax values */
    const float amax = f_of(b << 16);
    if (amax > 1e-12f) { scales[ns++] = amax / 127.0f; if (b % 7 == 0) scales[ns++] = amax / 448.0f; }
  }
  for (int i = 0; i < 150 && ns < 8190; ++i) {
    const float amax = ldexpf(1.0f + (float)(next_u32() & 0xffffff) / 16777216.0f, (int)(next_u32() % 40) - 20);
    scales[ns++] = amax / 127.0f;
  }
  for (int k = 0; k < ns; ++k) {
    const float s = scales[k];
    for (uint32_t b = 0; b < 0x10000u; ++b) {
      const float x = f_of(b << 16);
      if (isfinite(x)) check(x, s);
    }
  }
  for (int k = 0; k < ns; k += 5)
    for (int i = 0; i < 40000; ++i) {
      const float x = f_of(next_u32());
      if (isfinite(x)) check(x, scales[k]);
    }
  printf("checked %lld mismatches %lld\n", checked, bad);
  return bad != 0;
}
