// Division used by the vectorized INT8 quantizer (flashspec_amd/csrc/fs_common.h,
// div_by_scale): q1 = fma(fma(-q0, b, a), y, q0) with y = RN(1/b), q0 = RN(a*y).
// Compares q1 with IEEE a/b for every finite fp16 value a (and random fp32 values) over
// quantizer-like scales (mx - mn) / 255, all-ones significands and random normals, and
// prints the number of mismatches other than the sign of a zero quotient.
// Usage: markstein_check [n_scales] [n_random_fp32_per_scale]
#include <stdio.h>
#include <stdint.h>
#include <math.h>
#include <string.h>
#include <stdlib.h>
static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float half_to_f(uint16_t h) {
  uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) return NAN;
  else v = ldexpf((float)(m | 1024), (int)e - 25);
  return s ? -v : v;
}
static uint64_t rng = 88172645463325252ull;
static uint64_t xs() { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return rng; }
int main(int argc, char** argv) {
  const int n_scales = argc > 1 ? atoi(argv[1]) : 600, n_random = argc > 2 ? atoi(argv[2]) : 20000;
  long bad = 0, total = 0;
  for (int t = 0; t < n_scales; ++t) {
    float b;
    if (t < n_scales / 3) {  // scales as the quantizer makes them: (mx - mn) / 255 with random extremes
      float mx = (float)((xs() % 2000000) / 1000.0), mn = -(float)((xs() % 2000000) / 1000.0);
      b = fmaxf((mx - mn) / 255.0f, 1e-8f);
    } else if (t < 2 * n_scales / 3) {  // all-ones significands, many exponents
      b = f_of(((uint32_t)(100 + t % 60) << 23) | 0x7fffffu);
    } else {  // random positive normals
      b = f_of((uint32_t)((xs() % (200u << 23)) + (20u << 23)));
    }
    const float y = 1.0f / b;
    for (uint32_t h = 0; h < 65536; ++h) {
      const float a = half_to_f((uint16_t)h);
      if (isnan(a)) continue;
      const float ref = a / b;
      const float q0 = a * y;
      const float r = fmaf(-q0, b, a);
      const float q1 = fmaf(r, y, q0);
      ++total;
      if (u_of(q1) != u_of(ref) && !(q1 == 0.0f && ref == 0.0f) && !(isinf(ref) && isinf(q1))) {
        if (bad < 10) printf("mismatch a=%a b=%a ref=%a got=%a\n", a, b, ref, q1);
        ++bad;
      }
    }
    for (int k = 0; k < n_random; ++k) {  // random fp32 inputs in a wide range
      const float a = f_of((uint32_t)(xs() % (180u << 23)) + (40u << 23)) * ((xs() & 1) ? 1.f : -1.f);
      const float ref = a / b;
      if (isinf(ref) || ref == 0.0f || fabsf(ref) < 1e-37f) continue;
      const float q0 = a * y;
      const float r = fmaf(-q0, b, a);
      const float q1 = fmaf(r, y, q0);
      ++total;
      if (u_of(q1) != u_of(ref)) {
        if (bad < 10) printf("mismatch a=%a b=%a ref=%a got=%a\n", a, b, ref, q1);
        ++bad;
      }
    }
  }
  printf("total %ld bad %ld\n", total, bad);
  return bad != 0;
}
