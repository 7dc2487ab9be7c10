/* Exhaustive check of the division the quantize kernels use for a group with
 * a finite positive scale (iq_quant.hip, div_rcp): for every finite fp16
 * x >= 0 and every finite fp16 s > 0,
 *     RN16(q0 + RN32(x - q0 s) r)  with  r = RN32(1/s),  q0 = RN32(x r)
 * equals RN16(x / s), the reference's fp16 division (fp32 arithmetic, round
 * to nearest even; both fma steps fused).  Prints the pair count and the
 * mismatch count; exits 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

/* value of fp16 bit pattern h (h < 0x7c00: finite, >= 0) */
static float f16_value(uint32_t h) {
  const uint32_t e = h >> 10, m = h & 0x3ff;
  return e ? ldexpf((float)(m | 0x400), (int)e - 25) : ldexpf((float)m, -24);
}

/* x rounded to fp16 (nearest, ties to even), as fp32; x >= 0 or NaN */
static float round_f16(float x) {
  if (x != x) return x;
  if (x >= 65520.0f) return INFINITY;
  int e;
  frexpf(x, &e); /* x = f 2^e, f in [0.5, 1) */
  const int ue = (x < ldexpf(1.0f, -14)) ? -24 : e - 11; /* fp16 ulp exponent at x */
  return ldexpf(rintf(ldexpf(x, -ue)), ue);
}

int main(void) {
  static float val[0x7c00];
  for (uint32_t h = 0; h < 0x7c00; ++h) val[h] = f16_value(h);
  long long pairs = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad)
  for (int j = 1; j < 0x7c00; ++j) {
    const float s = val[j];
    const float r = 1.0f / s;
    for (int i = 0; i < 0x7c00; ++i) {
      const float x = val[i];
      const float q0 = x * r;
      const float q1 = fmaf(fmaf(-q0, s, x), r, q0);
      const float a = round_f16(q1), b = round_f16(x / s);
      ++pairs;
      if (memcmp(&a, &b, sizeof a) != 0) ++bad;
    }
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}
