/* Markstein-corrected division against IEEE division (the kernels' div_rt).
 *
 *   q0 = x * rt, r = fma(-t, q0, x), q1 = fma(r, rt, q0),
 *   rt = recip_rt(t) = RN(1 / t) for t in [2^-100, 2^100], else 0
 *
 * must equal RN(x / t) wherever the guard of div_rt lets it through
 * (|x|, |q0| in [2^-100, 2^100]).  RN(x / t) is computed in double and rounded
 * to float, which is correctly rounded for float operands (53 >= 2*24 + 2).
 * Usage: division_check <bf16 divisors> <float32 stride> <float32 divisors>
 * Prints "checked bad" for each part; exit status 1 when any case is bad.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float recip_rt(float t) { return (t >= 0x1p-100f && t <= 0x1p100f) ? 1.0f / t : 0.0f; }

static int same(float x, float t, float rt) {
  const float q0 = x * rt;
  const float aq = fabsf(q0);
  if (!(fabsf(x) >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f)) return 1; /* the division itself */
  const float r = fmaf(-t, q0, x);
  const float q1 = fmaf(r, rt, q0);
  return u_of(q1) == u_of((float)((double)x / (double)t));
}

static float divisor(long i) {
  if (i < 1000) return f_of(u_of(1.0f) + (uint32_t)i - 500u);                 /* around 1 */
  if (i < 2000) return ldexpf(1.0f + (float)(i % 7) * 1e-7f, (int)(i % 60) - 30); /* powers of two and neighbours */
  return 1e-8f + 10.0f * (float)((i * 2654435761u) % 1000003u) / 1000003.0f;  /* spread over (0, 10] */
}

int main(int argc, char** argv) {
  const long nb = argc > 1 ? atol(argv[1]) : 2000;
  const long stride = argc > 2 ? atol(argv[2]) : 97;
  const long nf = argc > 3 ? atol(argv[3]) : 2;
  long n = 0, bad = 0;
  for (long i = 0; i < nb; ++i) {
    const float t = divisor(i), rt = recip_rt(t);
    for (uint32_t p = 0; p < 65536; ++p) {
      const float x = f_of(p << 16);
      if (!isfinite(x)) continue;
      ++n;
      if (!same(x, t, rt)) { if (bad < 5) printf("bad bf16 x=%a t=%a\n", x, t); ++bad; }
    }
  }
  printf("bf16 %ld %ld\n", n, bad);
  /* divisors over the whole float range: 2^e times 5 mantissas, e in
     [-127, 127], and the neighbours of the recip_rt bounds */
  long nw = 0, badw = 0;
  const float ms[] = {1.0f, 1.0000001f, 1.3f, 1.7182818f, 1.9999999f};
  for (int e = -127; e <= 128; ++e) {
    for (int k = 0; k < 6; ++k) {
      float t;
      if (e == 128) t = k < 3 ? f_of(u_of(0x1p-100f) + (uint32_t)k - 1u) : f_of(u_of(0x1p100f) + (uint32_t)k - 4u);
      else if (k < 5) t = ldexpf(ms[k], e);
      else t = f_of(u_of(ldexpf(1.0f, e)) - 1u);
      if (!(t > 0.0f) || !isfinite(t)) continue;
      const float rt = recip_rt(t);
      for (uint32_t p = 0; p < 65536; ++p) {
        const float x = f_of(p << 16);
        if (!isfinite(x)) continue;
        ++nw;
        if (!same(x, t, rt)) { if (badw < 5) printf("bad wide x=%a t=%a\n", x, t); ++badw; }
      }
    }
  }
  printf("wide %ld %ld\n", nw, badw);
  const float ts[] = {0.8f, 0.7f, 1.3f, 0.1f, 1.5f, 0.123456f, 3.0f, 0.99999994f};
  long n32 = 0, bad32 = 0;
  for (long j = 0; j < nf && j < 8; ++j) {
    const float t = ts[j], rt = recip_rt(t);
    for (uint64_t u = (uint64_t)j; u < (1ull << 32); u += (uint64_t)stride) {
      const float x = f_of((uint32_t)u);
      if (!isfinite(x)) continue;
      ++n32;
      if (!same(x, t, rt)) { if (bad32 < 5) printf("bad f32 x=%a t=%a\n", x, t); ++bad32; }
    }
  }
  printf("f32 %ld %ld\n", n32, bad32);
  return (bad || bad32 || badw) ? 1 : 0;
}
