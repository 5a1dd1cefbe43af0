/* Exhaustive check of the quantiser's arithmetic (15642_moe_amd/csrc/upstream.hip,
 * quant_scale and quot).
 *
 * Scale: for every finite bf16 block amax m >= 0 (every value the row
 * maximum of bf16 elements can take), q0 = RN(m * c) with c = RN(1/448),
 * r = fma(-q0, 448, m), s = fma(r, c, q0) must equal RN(m / 448) bit for bit.
 *
 * Quotient: for every finite bf16 block amax a >= 0 in [lo, hi) (bf16 bit
 * patterns) and every bf16 x with |x| <= a, both signs,
 *   s  = max(RN(a / 448), 1e-8),  y = any float within 1 ulp of 1/s
 *        (RN(1/s) and its two neighbours: the kernel takes v_rcp_f32,
 *        documented as accurate to 1 ulp),
 *   q0 = RN(x * y),  r = fma(-q0, s, x),  q = copysign(fma(r, y, q0), x)
 * must give the same e4m3 code (RNE, after clamping to +-448) as the IEEE
 * quotient RN(x / s) that the reference rule (x / s, kernels/moe.cu:516-541)
 * and the oracle use.  The kernel passes s clamped to FLT_MAX to the
 * remainder FMA and guards the scale of an infinite amax; a block whose
 * amax is +inf is checked too, against every bf16 x including +-inf and NaN,
 * as is the scale of +inf and NaN.  Prints the counts; exits 1 if any scale or code
 * differs.  A third argument "plain" checks q = copysign(RN(x * RN(1/s)), x)
 * instead (no correction step), which the checker must reject.  Build:
 * gcc -O2 -ffp-contract=off ... -lm (no contraction: every operation above is
 * rounded on its own, as the GPU code issues them). */
#include <float.h>
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
/* RNE code of q clamped to +-448 as the kernel clamps, fminf(fmaxf(q, -448),
 * 448) (a NaN quotient becomes -448); ties go to the even code. */
static int e4m3_code(float q) {
  q = fminf(fmaxf(q, -448.f), 448.f);
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

  long long scale_diff = 0;
  const float c448 = 1.0f / 448.0f;
  for (int mb = 0; mb < 0x7F80; ++mb) {
    const float m = bf16((uint16_t)mb);
    const float q0 = m * c448;
    const float s = fmaf(fmaf(-q0, 448.0f, m), c448, q0);
    if (bits(s) != bits(m / 448.0f)) {
      if (scale_diff < 10) printf("scale differs: m=%a m/448=%a got=%a\n", m, m / 448.0f, s);
      ++scale_diff;
    }
  }

  {
    const float inf = INFINITY, nan = NAN;
    const float ms[2] = {inf, nan};
    for (int i = 0; i < 2; ++i) {  /* the kernel's guard: m <= FLT_MAX ? corrected : m */
      const float m = ms[i], q0 = m * c448;
      const float s = m <= FLT_MAX ? fmaf(fmaf(-q0, 448.0f, m), c448, q0) : m;
      const float want = m / 448.0f;
      if (!((isnan(s) && isnan(want)) || bits(s) == bits(want))) {
        printf("scale differs for non-finite m=%a\n", m);
        ++scale_diff;
      }
    }
  }

  long long cases = 0, code_diff = 0;
  for (int ab = lo; ab < hi && ab < 0x7F80; ++ab) {
    const float a = bf16((uint16_t)ab);
    const float s = fmaxf(a / 448.0f, 1e-8f);
    const float y_rn = 1.0f / s;
    const float ys[3] = {nextafterf(y_rn, 0.0f), y_rn, nextafterf(y_rn, INFINITY)};
    for (int xb = 0; xb <= ab; ++xb) {
      for (int neg = 0; neg < 2; ++neg) {
        const float x = bf16((uint16_t)(xb | (neg << 15)));
        const int want = e4m3_code(x / s);
        for (int k = plain ? 1 : 0; k < (plain ? 2 : 3); ++k) {
          const float y = ys[k];
          const float q0 = x * y;
          const float r = fmaf(-q0, fminf(s, FLT_MAX), x);
          const float q = plain ? copysignf(q0, x) : copysignf(fmaf(r, y, q0), x);
          ++cases;
          if (e4m3_code(q) != want) {
            if (code_diff < 10) printf("code differs: a=%a x=%a s=%a y=%a x/s=%a q=%a\n", a, x, s, y, x / s, q);
            ++code_diff;
          }
        }
      }
    }
  }
  if (hi >= 0x7F80 && !plain) {  /* amax +inf: s = inf, y = 1/inf = 0 exactly, every bf16 x */
    const float s = fmaxf(INFINITY / 448.0f, 1e-8f), y = 1.0f / s;
    for (int xb = 0; xb < 0x10000; ++xb) {
      const float x = bf16((uint16_t)xb);
      const float q0 = x * y;
      const float q = copysignf(fmaf(fmaf(-q0, fminf(s, FLT_MAX), x), y, q0), x);
      ++cases;
      if (e4m3_code(q) != e4m3_code(x / s)) {
        if (code_diff < 10) printf("code differs: a=inf x=%a x/s=%a q=%a\n", x, x / s, q);
        ++code_diff;
      }
    }
  }
  printf("scale: %lld differences; amax bits [%d, %d): %lld cases, %lld code differences\n", scale_diff, lo, hi,
         cases, code_diff);
  return scale_diff != 0 || code_diff != 0;
}
