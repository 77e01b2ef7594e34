// Accuracy of dpamd::tanh_fast (host build of the same source, with the
// hardware reciprocal seed modelled by rounding to fp32) against libm tanh
// over a dense grid, random points and powers of two; prints the max absolute
// error (the bound the network relies on) and, for information, the max
// error in ulp of the result.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "../../dpa4c-scale-aware-md_amd/csrc/fastmath.h"

static double ulp_err(double a, double b) {
  if (a == b) return 0.0;
  const double u = std::fabs(std::nextafter(b, INFINITY) - b);
  return std::fabs(a - b) / (u > 0 ? u : 1e-300);
}

int main() {
  double max_ulp = 0, max_abs = 0, worst = 0;
  std::mt19937_64 g(7);
  std::uniform_real_distribution<double> U(-25.0, 25.0);
  auto check = [&](double x) {
    const double a = dpamd::tanh_fast(x), b = std::tanh(x);
    const double e = ulp_err(a, b);
    if (e > max_ulp) { max_ulp = e; worst = x; }
    if (std::fabs(a - b) > max_abs) max_abs = std::fabs(a - b);
  };
  for (int i = -2000000; i <= 2000000; ++i) check(i * 1e-5);
  for (int i = 0; i < 2000000; ++i) check(U(g));
  for (int k = -300; k < 3; ++k) { check(std::ldexp(1.0, k)); check(-std::ldexp(1.3, k)); }
  check(0.0);
  std::printf("max_ulp %.3f at x=%.17g max_abs %.3e\n", max_ulp, worst, max_abs);
  // four at a time (shared reciprocal): mixed magnitudes, including the clamp
  double max_abs4 = 0;
  std::uniform_real_distribution<double> W(-1.0, 1.0);
  for (int i = 0; i < 2000000; ++i) {
    double x[4], y[4];
    for (int k = 0; k < 4; ++k) x[k] = (i % 3 == 0) ? U(g) : W(g) * std::pow(10.0, (i % 7) - 4);
    if (i % 11 == 0) x[i % 4] = (i % 2 ? 25.0 : -30.0);
    if (i % 13 == 0) x[(i + 1) % 4] = 0.0;
    dpamd::tanh_fast4(x, y);
    for (int k = 0; k < 4; ++k) max_abs4 = std::fmax(max_abs4, std::fabs(y[k] - std::tanh(x[k])));
  }
  double z4[4], zx[4] = {0.0, -0.0, 0.0, 0.0};
  dpamd::tanh_fast4(zx, z4);
  const bool zeros = z4[0] == 0.0 && z4[1] == 0.0;
  std::printf("tanh_fast4 max_abs %.3e, tanh(0) exact %d\n", max_abs4, (int)zeros);
  // table-driven form (the embedding kernels): dense grid, random mixed
  // magnitudes, the clamp, exact zeros and odd symmetry
  double max_tab = 0;
  auto tab4 = [&](const double* x) {
    double y[4];
    dpamd::tanh_tab4(x, y, dpamd::kTanhTab32);
    for (int k = 0; k < 4; ++k) max_tab = std::fmax(max_tab, std::fabs(y[k] - std::tanh(x[k])));
  };
  for (int i = -2000000; i <= 2000000; i += 4) {
    const double x[4] = {i * 1e-5, (i + 1) * 1e-5, (i + 2) * 1e-5, (i + 3) * 1e-5};
    tab4(x);
  }
  for (int i = 0; i < 2000000; ++i) {
    double x[4];
    for (int k = 0; k < 4; ++k) x[k] = (i % 3 == 0) ? U(g) : W(g) * std::pow(10.0, (i % 7) - 4);
    if (i % 11 == 0) x[i % 4] = (i % 2 ? 25.0 : -30.0);
    if (i % 13 == 0) x[(i + 1) % 4] = 0.0;
    tab4(x);
  }
  double t4[4], tx[4] = {0.0, -0.0, 1e-300, -3.0}, tn[4], txn[4] = {0.0, 0.0, -1e-300, 3.0};
  dpamd::tanh_tab4(tx, t4, dpamd::kTanhTab32);
  dpamd::tanh_tab4(txn, tn, dpamd::kTanhTab32);
  const bool tzero = t4[0] == 0.0 && t4[1] == 0.0 && std::signbit(t4[1]) && t4[3] == -tn[3];
  std::printf("tanh_tab4 max_abs %.3e, zeros / odd symmetry %d\n", max_tab, (int)tzero);
  // one value at a time (the embedding kernels' lone tail features)
  double max_tab1 = 0;
  auto tab1 = [&](double x) {
    max_tab1 = std::fmax(max_tab1, std::fabs(dpamd::tanh_tab1(x, dpamd::kTanhTab32) - std::tanh(x)));
  };
  for (int i = -2000000; i <= 2000000; ++i) tab1(i * 1e-5);
  for (int i = 0; i < 2000000; ++i) tab1((i % 3 == 0) ? U(g) : W(g) * std::pow(10.0, (i % 7) - 4));
  tab1(25.0);
  tab1(-30.0);
  const double o0 = dpamd::tanh_tab1(0.0, dpamd::kTanhTab32), o1 = dpamd::tanh_tab1(-0.0, dpamd::kTanhTab32);
  const bool t1zero = o0 == 0.0 && o1 == 0.0 && std::signbit(o1) &&
                      dpamd::tanh_tab1(-3.0, dpamd::kTanhTab32) == -dpamd::tanh_tab1(3.0, dpamd::kTanhTab32);
  std::printf("tanh_tab1 max_abs %.3e, zeros / odd symmetry %d\n", max_tab1, (int)t1zero);
  return (max_abs <= 4e-15 && max_abs4 <= 4e-15 && zeros && max_tab <= 4e-15 && tzero &&
          max_tab1 <= 4e-15 && t1zero)
             ? 0
             : 1;
}
