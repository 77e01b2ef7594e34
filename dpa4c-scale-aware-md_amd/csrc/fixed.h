// Order-independent force / atom-virial accumulation in 64-bit fixed point.
//
// Each edge's contribution to its target atom is rounded once to a signed
// integer in units of 2^-40 and added with a 64-bit integer atomic. Integer
// addition is associative, so the totals do not depend on the order in which
// waves arrive (bit-reproducible) and no reverse neighbour list is needed.
// The reference accumulates its split forces the same way in fixed point
// (deepmd-op/overlays/op/pt/dpa4c/raw_force_split.cuh:302-312, 24 fraction
// bits for its fp32 model); 40 bits keep this library's fp64 path exact to
// 2^-41 = 4.5e-13 per term (176 terms into one Cu atom: below 1e-10 eV/A),
// with a range of +-2^23 = 8.4e6 per accumulated value. Each term must stay
// below 2^11 = 2048 in magnitude (the conversion's range), so up to kFixTerms
// = 4096 terms into one atom cannot wrap; the callers keep force terms (edge
// gradient components) below 2^11 and virial terms (g (x) d with |d| <= rcut)
// below that times the cutoff radius, and raise a status flag otherwise.
#pragma once

#include "common.h"

namespace dpamd {

constexpr double kFixInv = 0x1p-40;
constexpr double kFixTerms = 4096.0;  // terms into one atom the range allows
constexpr double kFixTermMax = 0x1p11;  // exclusive bound of one term

// Largest |edge-gradient component| whose force and virial terms stay inside
// the conversion's range (rcut in A; the factor keeps the rounded products
// strictly below kFixTermMax).
inline double fixed_gmax(double rcut) {
  return kFixTermMax * (1.0 - 0x1p-20) / (rcut > 1.0 ? rcut : 1.0);
}

// round(x * 2^40) (ties to even) as a two's complement 64-bit pattern, exact
// for |x| < 2^11: adding C = 1.5 * 2^12, whose ulp is 2^-40, rounds x to a
// multiple of 2^-40 and, the sum staying in [2^12, 2^13), leaves
// 2^51 + round(x * 2^40) in the significand field, so subtracting the bit
// pattern of C leaves round(x * 2^40). One fp64 add and one 64-bit integer
// subtract.
__device__ __forceinline__ unsigned long long to_fixed(double x) {
  constexpr double kC = 0x1.8p12;
  return __builtin_bit_cast(unsigned long long, x + kC) -
         __builtin_bit_cast(unsigned long long, kC);
}

__device__ __forceinline__ double from_fixed(unsigned long long k) {
  const int hi = (int)(k >> 32);
  const unsigned lo = (unsigned)(k & 0xffffffffull);
  return ((double)hi * 0x1p32 + (double)lo) * kFixInv;
}

__device__ __forceinline__ void fixed_add(unsigned long long* p, double x) {
  atomicAdd(p, to_fixed(x));
}

}  // namespace dpamd
