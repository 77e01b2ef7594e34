// Hyperbolic tangent for the network kernels, fp64 and fp32.
//
// fp64 (written from the mathematics, not from any vendor library):
//   tanh|x| = 1 - 2 / (2^t + 1),   t = 2|x| log2(e)
//   2^t = 2^n 2^f with n = rint(t), f = t - n (exact), |f| <= 1/2;
//   2^f by a degree-10 polynomial interpolating 2^f at the 11 Chebyshev
//     nodes of [-1/2, 1/2] (coefficients computed in extended precision and
//     rounded, the constant term to exactly 1; max relative error below
//     2e-15 on the interval);
//   1/(2^t + 1) from the hardware reciprocal seed (about 24 bits) refined by
//     one Newton step z <- z + z(1 - d z) (about 48 bits).
// |x| is clamped at 20 (tanh(20) rounds to 1). The error is absolute, not
// relative: at most about 3e-15 over the real line (tests/test_native.py),
// which is what the network needs (activations enter sums of O(1) terms) and
// four orders of magnitude below what the fp64 energy/force tolerances can
// see; near 0 the relative error is therefore large. Cost: 22 VALU
// operations, against about 32 for an expm1-based form with full relative
// accuracy.
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
  // host model of a reduced-precision seed: the quotient with its significand
  // rounded to 24 bits (exponent range of fp64 kept)
  int e;
  const double m = std::frexp(1.0 / d, &e);
  return std::ldexp((double)(float)m, e);
#endif
}

// 2^t + 1 for t = 2|x| log2(e), |x| clamped at 20 (so the result is below
// 2^58): the denominator of tanh|x| = 1 - 2 / (2^t + 1).
DPAMD_HD inline double tanh_denominator(double x) {
  const double ax = fmin(fabs(x), 20.0);
  const double t = ax * 2.8853900817779268;  // 2 log2(e)
  const double n = rint(t);
  const double f = t - n;
  double p = 6.881851856054378e-09;
  p = fma(p, f, 1.020195864756798e-07);
  p = fma(p, f, 1.3216503079020598e-06);
  p = fma(p, f, 1.5252692473004133e-05);
  p = fma(p, f, 0.00015403528490158397);
  p = fma(p, f, 0.0013333558169839458);
  p = fma(p, f, 0.009618129108904515);
  p = fma(p, f, 0.05550410866482973);
  p = fma(p, f, 0.24022650695907963);
  p = fma(p, f, 0.6931471805599428);
  p = fma(p, f, 1.0);  // interpolant value 1 + 2.2e-16, rounded to 1 so tanh(0) = 0
  return ldexp(p, (int)n) + 1.0;
}

// Four tanh at once sharing one reciprocal (Montgomery's trick): with
// P = d0 d1 d2 d3 (< 2^232), 1/P from the seed and one Newton step, then
// 1/(d0 d1) = P^-1 d2 d3, 1/d0 = 1/(d0 d1) d1, and so on. The hardware
// reciprocal costs about 3.4 FMAs of issue time on gfx950, so this saves ~7
// FMA-equivalents per four values; the extra roundings keep the absolute
// error within the same bound as tanh_fast (tests/test_native.py).
DPAMD_HD inline void tanh_fast4(const double x[4], double y[4]) {
  double d[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) d[k] = tanh_denominator(x[k]);
  const double p01 = d[0] * d[1], p23 = d[2] * d[3], P = p01 * p23;
  double r = rcp_seed(P);
  r = fma(fma(-P, r, 1.0), r, r);
  const double r01 = r * p23, r23 = r * p01;
  const double z[4] = {r01 * d[1], r01 * d[0], r23 * d[3], r23 * d[2]};
#pragma unroll
  for (int k = 0; k < 4; ++k) y[k] = copysign(fma(-2.0, z[k], 1.0), x[k]);
}

DPAMD_HD inline double tanh_fast(double x) {
  const double ax = fmin(fabs(x), 20.0);
  const double t = ax * 2.8853900817779268;  // 2 log2(e)
  const double n = rint(t);
  const double f = t - n;
  double p = 6.881851856054378e-09;
  p = fma(p, f, 1.020195864756798e-07);
  p = fma(p, f, 1.3216503079020598e-06);
  p = fma(p, f, 1.5252692473004133e-05);
  p = fma(p, f, 0.00015403528490158397);
  p = fma(p, f, 0.0013333558169839458);
  p = fma(p, f, 0.009618129108904515);
  p = fma(p, f, 0.05550410866482973);
  p = fma(p, f, 0.24022650695907963);
  p = fma(p, f, 0.6931471805599428);
  p = fma(p, f, 1.0);  // interpolant value 1 + 2.2e-16, rounded to 1 so tanh(0) = 0
  const double d = ldexp(p, (int)n) + 1.0;
  double z = rcp_seed(d);
  z = fma(fma(-d, z, 1.0), z, z);
  return copysign(fma(-2.0, z, 1.0), x);
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
