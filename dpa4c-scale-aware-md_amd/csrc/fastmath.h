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

// Table-driven fp64 tanh, four at a time (the embedding kernels):
//   tanh|x| = (1 - e) / (1 + e),  e = 2^-t,  t = 2|x| log2(e)
// with |x| clamped at 20 as above; the negative exponent keeps 1 + e in
// (1, 2], so the product of four denominators cannot overflow, and
// tanh(0) = 0 exactly (e = 1). With 128 t = k + f' (k = rint, |f'| <= 1/2),
// k = 128 n + j (j = 0..127):
//   e = 2^n * 2^(j/128) * p(f'),  p(f') = 2^(f'/128) = 1 + f' q(f')
// where 2^(j/128) comes from a 128-entry table (kExp2Tab128, correctly
// rounded; the kernels keep it in LDS) and q is the cubic interpolating
// (2^(f'/128) - 1) / f' at the Chebyshev nodes (fastmath_coeffs.py derives
// both). rint uses the 1.5 * 2^52 shifter, whose low word then holds k; 2^n
// is added to the exponent field directly (n in [-58, 0]: the result stays
// normal). Cost: 16 fp64 operations (three of them the shared reciprocal's
// share), 5 integer operations and one LDS read per value, against 21 fp64
// for tanh_fast4; absolute error within 4e-15 (tests/native/tanh_check.cpp).
constexpr double kExp2Tab128[128] = {
    1.0, 1.0054299011128027, 1.0108892860517005, 1.016378314910953,
    1.0218971486541166, 1.0274459491187637, 1.0330248790212284, 1.0386341019613787,
    1.0442737824274138, 1.0499440858006872, 1.0556451783605572, 1.061377227289262,
    1.0671404006768237, 1.0729348675259756, 1.0787607977571199, 1.0846183622133092,
    1.0905077326652577, 1.0964290818163769, 1.102382583307841, 1.1083684117236787,
    1.1143867425958924, 1.1204377524096067, 1.1265216186082418, 1.1326385195987192,
    1.1387886347566916, 1.1449721444318042, 1.1511892299529827, 1.1574400736337511,
    1.1637248587775775, 1.1700437696832502, 1.1763969916502812, 1.182784710984341,
    1.189207115002721, 1.1956643920398273, 1.202156731452703, 1.2086843236265816,
    1.215247359980469, 1.2218460329727576, 1.22848053610687, 1.2351510639369334,
    1.241857812073484, 1.2486009771892048, 1.255380757024691, 1.2621973503942507,
    1.2690509571917332, 1.275941778396392, 1.2828700160787783, 1.2898358734066657,
    1.2968395546510096, 1.3038812651919358, 1.3109612115247644, 1.318079601266064,
    1.3252366431597413, 1.3324325470831615, 1.339667524053303, 1.3469417862329458,
    1.3542555469368927, 1.3616090206382248, 1.3690024229745905, 1.3764359707545302,
    1.383909881963832, 1.3914243757719262, 1.3989796725383112, 1.4065759938190154,
    1.4142135623730951, 1.4218926021691656, 1.42961333839197, 1.4373759974489824,
    1.4451808069770467, 1.4530279958490526, 1.460917794180647, 1.4688504333369818,
    1.4768261459394993, 1.4848451658727524, 1.4929077282912648, 1.5010140696264256,
    1.5091644275934228, 1.5173590411982147, 1.5255981507445384, 1.533881997840956,
    1.5422108254079407, 1.550584877685, 1.559004400237837, 1.567469639965553,
    1.5759808451078865, 1.5845382652524937, 1.593142151342267, 1.6017927556826934,
    1.6104903319492543, 1.6192351351948637, 1.6280274218573478, 1.6368674497669644,
    1.645755478153965, 1.6546917676561943, 1.6636765803267364, 1.6727101796415966,
    1.681792830507429, 1.6909247992693053, 1.7001063537185235, 1.709337763100463,
    1.718619298122478, 1.7279512309618377, 1.7373338352737062, 1.746767386199169,
    1.7562521603732995, 1.7657884359332727, 1.7753764925265212, 1.785016611318935,
    1.7947090750031072, 1.804454167806624, 1.8142521755003989, 1.8241033854070534,
    1.8340080864093424, 1.843966568958626, 1.8539791250833855, 1.864046048397789,
    1.8741676341103, 1.8843441790323345, 1.8945759815869656, 1.9048633418176741,
    1.9152065613971474, 1.925605943636125, 1.9360617934922943, 1.9465744175792332,
    1.9571441241754002, 1.9677712232331759, 1.978456026387951, 1.9891988469672663,
};
constexpr double kTabQ1 = 0.00541521234812427, kTabQ2 = 1.466226238764015e-05;
constexpr double kTabQ3 = 2.6466431145772844e-08, kTabQ4 = 3.5830331809896814e-11;

// e = 2^(-2 |x| log2 e) for |x| clamped at 20
DPAMD_HD inline double tab_exp(double x, const double* tab) {
  const double t = fmin(fabs(x), 20.0) * -369.32993046757463;  // -256 log2(e) |x|
  const double sh = t + 6755399441055744.0;                     // 1.5 * 2^52
  const double kf = sh - 6755399441055744.0;
  const double f = t - kf;
  const int k = (int)(unsigned)__builtin_bit_cast(unsigned long long, sh);
  const double T = tab[k & 127];
  const int n = k >> 7;
  double q = fma(kTabQ4, f, kTabQ3);
  q = fma(q, f, kTabQ2);
  q = fma(q, f, kTabQ1);
  const double e0 = fma(f, q, 1.0) * T;
  // 2^n into the exponent field (the low word is untouched)
  return __builtin_bit_cast(double, __builtin_bit_cast(unsigned long long, e0) +
                                        ((unsigned long long)(long long)n << 52));
}

DPAMD_HD inline void tanh_tab4(const double x[4], double y[4], const double* tab) {
  double e[4], d[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    e[k] = tab_exp(x[k], tab);
    d[k] = 1.0 + e[k];
  }
  const double p01 = d[0] * d[1], p23 = d[2] * d[3], P = p01 * p23;
  double r = rcp_seed(P);
  r = fma(fma(-P, r, 1.0), r, r);
  const double r01 = r * p23, r23 = r * p01;
  const double z[4] = {r01 * d[1], r01 * d[0], r23 * d[3], r23 * d[2]};
#pragma unroll
  for (int k = 0; k < 4; ++k) y[k] = copysign((1.0 - e[k]) * z[k], x[k]);
}

DPAMD_HD inline double tanh_act(double x) { return tanh_fast(x); }
DPAMD_HD inline float tanh_act(float x) { return tanh_f32(x); }

}  // namespace dpamd
