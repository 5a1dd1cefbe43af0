/* Exhaustive check of the quantiser's division (15642_moe_amd/csrc/upstream.hip,
 * quot): for every finite bf16 block amax a >= 0 in [lo, hi) (bf16 bit
 * patterns) and every bf16 x with |x| <= a, both signs,
 *   s  = max(RN(a / 448), 1e-8),  y = RN(1 / s),
 *   q0 = RN(x * y),  r = fma(-q0, s, x),  q = copysign(fma(r, y, q0), x)
 * must give the same e4m3 code (RNE, after clamping to +-448) as the IEEE
 * quotient RN(x / s) that the reference rule (x / s, kernels/moe.cu:516-541)
 * and the oracle use.  Prints the pair count, the number of pairs whose
 * quotients differ in any bit and the number whose codes differ; exits 1 if
 * any code differs.  A third argument "plain" checks q = copysign(RN(x * y), x)
 * instead (no correction step), which the checker must reject.  Build:
 * gcc -O2 -ffp-contract=off ... -lm (no contraction: every operation above is
 * rounded on its own, as the GPU code issues them). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* e4m3 (bias 7, no infinities, 0x7F = NaN): the 127 non-negative values. */
static double e4m3_value[127];
static double e4m3_decode(int c) {
  const int e = (c >> 3) & 15, m = c & 7;
  return e ? ldexp(1.0 + m / 8.0, e - 7) : ldexp(m / 8.0, -6);
}
/* RNE code of q clamped to +-448; ties go to the even code. */
static int e4m3_code(float q) {
  if (q > 448.f) q = 448.f;
  if (q < -448.f) q = -448.f;
  const int sign = signbit(q) ? 0x80 : 0;
  const double a = fabs((double)q);
  int lo = 0, hi = 126; /* e4m3_value[lo] <= a <= e4m3_value[hi] */
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (e4m3_value[mid] <= a) lo = mid;
    else hi = mid;
  }
  int c;
  if (a == e4m3_value[lo]) c = lo;
  else if (a == e4m3_value[hi]) c = hi;
  else {
    const double dl = a - e4m3_value[lo], dh = e4m3_value[hi] - a;
    c = dl < dh ? lo : dh < dl ? hi : ((lo & 1) ? hi : lo);
  }
  return sign | c;
}

int main(int argc, char** argv) {
  for (int c = 0; c < 127; ++c) e4m3_value[c] = e4m3_decode(c);
  const int lo = argc > 1 ? atoi(argv[1]) : 0, hi = argc > 2 ? atoi(argv[2]) : 0x7F80;
  const int plain = argc > 3 && strcmp(argv[3], "plain") == 0;
  long long pairs = 0, quotient_diff = 0, code_diff = 0;
  for (int ab = lo; ab < hi && ab < 0x7F80; ++ab) {
    const float a = bf16((uint16_t)ab);
    const float s = fmaxf(a / 448.0f, 1e-8f);
    const float y = 1.0f / s;
    for (int xb = 0; xb <= ab; ++xb) {
      for (int neg = 0; neg < 2; ++neg) {
        const float x = bf16((uint16_t)(xb | (neg << 15)));
        const float ref = x / s;
        const float q0 = x * y;
        const float r = fmaf(-q0, s, x);
        const float q = plain ? copysignf(q0, x) : copysignf(fmaf(r, y, q0), x);
        ++pairs;
        if (bits(q) == bits(ref)) continue;
        ++quotient_diff;
        if (e4m3_code(q) != e4m3_code(ref)) {
          if (code_diff < 10) printf("code differs: a=%a x=%a s=%a x/s=%a q=%a\n", a, x, s, ref, q);
          ++code_diff;
        }
      }
    }
  }
  printf("amax bits [%d, %d): %lld pairs, %lld quotient differences, %lld code differences\n", lo, hi, pairs,
         quotient_diff, code_diff);
  return code_diff != 0;
}
