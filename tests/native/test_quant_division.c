/* Exhaustive check of the activation-quantization division used by the HIP
 * kernels (CPU, no GPU).
 *
 * The W8A8 activation quantization (w8a8.py:8-14) computes, per 128-group of
 * a bf16 or fp16 row, s = fl(max(amax, 1e-10) * fl(1/127)) and
 * q = rint(x / s) with a correctly rounded fp32 division.  The kernels divide
 * every element by the same s, so they take r = fl(1 / s) once per group
 * (one correctly rounded division) and form each quotient as
 *     y = fl(x * r);  e = fma(-y, s, x);  q' = fma(e, r, y)
 * (one multiply and two fused multiply-adds: Markstein's correction step).
 * This program checks, for every finite bf16 and fp16 value a >= 0 as the
 * group absmax and every value x of the same type with |x| <= a, that
 * rint(q') equals rint(x / s), the value the int8 cast takes.  Both
 * operations are IEEE round-to-nearest-even in fp32 with denormals, as on the
 * GPU.  q' itself equals the correctly rounded quotient for every fp16 pair;
 * for bf16 it differs only where x is tiny (|x| < 2^-110) and the residual e
 * falls into the denormal range, and there the quotient is below 2^-70, so
 * both round to 0.  Those pairs are counted and that bound is checked too.
 *
 * Build: cc -O2 -ffp-contract=off [-fopenmp] test_quant_division.c -lm
 * Prints "division ok" and exits 0 when every pair agrees.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f32_of_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits_of_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* value of a 16-bit pattern of the given type (0: bf16, 1: fp16) */
static float decode16(int type, uint32_t h) {
  if (type == 0) return f32_of_bits(h << 16);
  const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 31u, man = h & 1023u;
  float v;
  if (ex == 0)
    v = ldexpf((float)man, -24); /* denormal: man * 2^-24, exact */
  else
    v = ldexpf((float)(man | 1024u), (int)ex - 25);
  return sign ? -v : v;
}

static int is_finite16(int type, uint32_t h) {
  return type == 0 ? ((h >> 7) & 0xFFu) != 0xFFu : ((h >> 10) & 31u) != 31u;
}

int main(void) {
  const float inv127 = (float)(1.0 / 127.0);
  long long total = 0, bad = 0, inexact = 0;
  for (int type = 0; type < 2; ++type) {
    /* magnitudes: non-negative patterns below the sign bit, ascending value */
    static float mag[32768];
    int n = 0;
    for (uint32_t h = 0; h < 0x8000u; ++h)
      if (is_finite16(type, h)) mag[n++] = decode16(type, h);
    long long t_total = 0, t_bad = 0, t_inexact = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : t_total, t_bad, t_inexact)
    for (int ia = 0; ia < n; ++ia) {
      const float a = mag[ia];
      const float s = fmaxf(a, 1e-10f) * inv127;
      const float r = 1.0f / s;
      for (int ix = 0; ix <= ia; ++ix) {
        for (int sg = 0; sg < 2; ++sg) {
          const float x = sg ? -mag[ix] : mag[ix];
          const float ref = x / s;
          const float y = x * r;
          const float e = fmaf(-y, s, x);
          const float q = fmaf(e, r, y);
          ++t_total;
          if (rintf(q) != rintf(ref)) ++t_bad;
          if (bits_of_f32(q) != bits_of_f32(ref) && !(q == 0.0f && ref == 0.0f)) {
            ++t_inexact;
            /* only tiny x, and far below the first rounding boundary */
            if (fabsf(x) >= 0x1p-110f || fabsf(ref) >= 0x1p-70f) ++t_bad;
          }
        }
      }
    }
    printf("%s: %lld pairs, %lld mismatches, %lld tiny inexact quotients\n",
           type == 0 ? "bf16" : "fp16", t_total, t_bad, t_inexact);
    total += t_total;
    bad += t_bad;
    inexact += t_inexact;
  }
  if (bad == 0) {
    printf("division ok (%lld pairs, %lld tiny inexact quotients)\n", total, inexact);
    return 0;
  }
  return 1;
}
