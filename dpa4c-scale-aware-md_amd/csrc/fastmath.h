// Hyperbolic tangent for the network kernels, fp64 and fp32.
//
// fp64:
// Method (written from the mathematics, not from any vendor library):
//   tanh(x) = sign(x) * E / (E + 2),  E = expm1(2|x|)
//   expm1(y) = 2^n (expm1(r) + 1) - 1 with Cody-Waite reduction
//     n = rint(y / ln2), r = (y - n*ln2_hi) - n*ln2_lo   (W. J. Cody and
//     W. Waite, Software Manual for the Elementary Functions, 1980),
//     ln2_hi = ln 2 rounded to 33 significant bits (n*ln2_hi exact), ln2_lo
//     the remainder, |r| <= ln2/2;
//   expm1(r) = r + r^2 (1/2! + r/3! + ... + r^11/13!)  (Taylor series; the
//     truncation term r^14/14! < 5e-18 for |r| <= ln2/2);
//   1/(E+2) from the hardware reciprocal seed refined by two Newton steps
//     z <- z + z(1 - d z), quadratically convergent.
// |x| is clamped at 20 (tanh(20) rounds to 1 in fp64). Measured error against
// libm is a few ulp (tests/test_native.py).
//
// fp32 (mixed-precision nets): tanh|x| = 1 - 2 / (e^{2|x|} + 1) with the
// hardware base-2 exponential and reciprocal (v_exp_f32, v_rcp_f32, each
// about 1 ulp). The formula cancels near 0, so the error is absolute rather
// than relative: at most 1.2e-7 against fp64 tanh over [-12, 12] when both
// hardware operations are correctly rounded (checked on the host), the same
// order as rounding an O(1) activation to fp32. e^{2|x|} overflows to +inf
// for |x| > 44, which gives exactly 1.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#define DPAMD_HD __host__ __device__
#else
#define DPAMD_HD
#endif

namespace dpamd {

DPAMD_HD inline double rcp_seed(double d) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_rcp(d);
#else
  // host model of a reduced-precision seed: round the quotient to fp32
  return (double)(float)(1.0 / d);
#endif
}

DPAMD_HD inline double tanh_fast(double x) {
  const double ax = fmin(fabs(x), 20.0);
  const double y = ax + ax;
  const double n = rint(y * 1.4426950408889634);
  const double r = fma(-n, 7.440617110012397e-11, fma(-n, 0.6931471804855391, y));
  double p = 1.6059043836821613e-10;
  p = fma(p, r, 2.08767569878681e-09);
  p = fma(p, r, 2.505210838544172e-08);
  p = fma(p, r, 2.755731922398589e-07);
  p = fma(p, r, 2.7557319223985893e-06);
  p = fma(p, r, 2.48015873015873e-05);
  p = fma(p, r, 0.0001984126984126984);
  p = fma(p, r, 0.001388888888888889);
  p = fma(p, r, 0.008333333333333333);
  p = fma(p, r, 0.041666666666666664);
  p = fma(p, r, 0.16666666666666666);
  p = fma(p, r, 0.5);
  const double em = fma(p, r * r, r);              // expm1(r)
  const double s = ldexp(1.0, (int)n);             // 2^n, exact
  const double E = fma(s, em, s - 1.0);            // expm1(y)
  const double d = E + 2.0;
  double z = rcp_seed(d);
  z = fma(fma(-d, z, 1.0), z, z);
  z = fma(fma(-d, z, 1.0), z, z);
  return copysign(E * z, x);
}

DPAMD_HD inline float tanh_f32(float x) {
  const float t = fabsf(x) * 2.8853900817779268f;  // 2|x| log2(e)
#if defined(__HIP_DEVICE_COMPILE__)
  const float e = __builtin_amdgcn_exp2f(t);
  const float y = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
#else
  const float e = exp2f(t);
  const float y = fmaf(-2.0f, 1.0f / (e + 1.0f), 1.0f);
#endif
  return copysignf(y, x);
}

DPAMD_HD inline double tanh_act(double x) { return tanh_fast(x); }
DPAMD_HD inline float tanh_act(float x) { return tanh_f32(x); }

}  // namespace dpamd
