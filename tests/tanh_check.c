/* The kernels' polynomial tanh (fl_tanh in csrc/fl_device.h) against tanh.
 *
 *   t = z * z, p = P(t) by Horner's rule in FMAs, tanh(z) ~ fma(z * t, p, z)
 *
 * over the float32 values z in [0, 0.625) (every stride-th bit pattern; the
 * odd form gives the negative half by symmetry).  The reference value is
 * double-precision tanh rounded to float.  Usage:
 *   tanh_check <stride> <p0> <p1> <p2> <p3> <p4> <p5>
 * Every sampled value is also compared with the polynomial at the next
 * float up (a decrease between neighbours is counted), and the polynomial's
 * value at the largest float below 0.625 -- where the kernels switch to
 * tanhf, which they floor at this value -- is printed in hex.
 * Prints "checked <n> differ <n> max_err_ulp <e> decreases <n> switch <hex>".
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float P[6];

static float poly(float z) {
  const float t = z * z;
  float p = fmaf(t, P[5], P[4]);
  p = fmaf(t, p, P[3]);
  p = fmaf(t, p, P[2]);
  p = fmaf(t, p, P[1]);
  p = fmaf(t, p, P[0]);
  return fmaf(z * t, p, z);
}

int main(int argc, char** argv) {
  if (argc != 8) return 2;
  const uint32_t stride = (uint32_t)strtoul(argv[1], NULL, 10);
  for (int i = 0; i < 6; ++i) P[i] = strtof(argv[2 + i], NULL);
  long n = 0, differ = 0, decreases = 0;
  double max_err = 0.0;
  float prev = 0.0f;
  for (uint32_t u = 0; f_of(u) < 0.625f; u += stride) {
    const float z = f_of(u);
    const float r = poly(z);
    if (f_of(u + 1) < 0.625f && poly(f_of(u + 1)) < r) ++decreases;
    const double ref = tanh((double)z);
    const float rf = (float)ref;
    if (u_of(r) != u_of(rf)) ++differ;
    if (rf > 0.0f) {
      const double ulp = (double)nextafterf(rf, 1.0f) - (double)rf;
      const double e = fabs((double)r - ref) / ulp;
      if (e > max_err) max_err = e;
    }
    if (r < prev) ++decreases;
    prev = r;
    ++n;
  }
  printf("checked %ld differ %ld max_err_ulp %.4f decreases %ld switch 0x%08x\n", n, differ, max_err, decreases,
         u_of(poly(nextafterf(0.625f, 0.0f))));
  return 0;
}
