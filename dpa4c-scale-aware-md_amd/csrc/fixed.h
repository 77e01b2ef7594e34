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
// with a range of +-2^23 = 8.4e6 per accumulated value. The callers keep each
// term below 2^23 / kFixTerms (forces) or that over the cutoff radius
// (virials, whose terms are g (x) d with |d| <= rcut) and raise a status flag
// otherwise, so that up to kFixTerms terms into one atom cannot wrap.
#pragma once

#include "common.h"

namespace dpamd {

constexpr double kFixScale = 0x1p40;
constexpr double kFixInv = 0x1p-40;
constexpr double kFixTerms = 1024.0;  // terms into one atom the range check assumes

// Largest |edge-gradient component| whose force and virial terms keep
// kFixTerms of them inside the range (rcut in A).
inline double fixed_gmax(double rcut) { return 0x1p23 / kFixTerms / (rcut > 1.0 ? rcut : 1.0); }

// round(x * 2^40) as a two's complement 64-bit pattern; exact for
// |x| < 2^23 (the high word from floor(y / 2^32), the low word the exact
// remainder in [0, 2^32)).
__device__ __forceinline__ unsigned long long to_fixed(double x) {
  const double y = rint(x * kFixScale);
  const double hi = floor(y * 0x1p-32);
  const double lo = fma(hi, -0x1p32, y);
  return ((unsigned long long)(unsigned)(int)hi << 32) | (unsigned long long)(unsigned)lo;
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
