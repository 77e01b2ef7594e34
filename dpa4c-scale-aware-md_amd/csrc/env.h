// Environment row of one neighbour slot and its gradient, in fp64 (both
// precision modes compute the env matrix, the edge gradient and everything
// downstream of it in fp64), plus the (ti, tj) pair lookup of the embedding
// kernels' block table.
#pragma once

#include "fixed.h"
#include "kernels.h"

namespace dpamd {

// The kernels keep a pair's env statistics as avg[4] and isd[4] = 1 / dstd
// (staged once per block), and EmbArgs carries inv_sw = 1 / (rcut -
// rcut_smth), so no IEEE division is left per slot; 1/r comes from the
// hardware reciprocal square root refined by two Newton steps (relative
// error at the rounding level). The oracle divides; the two agree to a few
// ulp, far inside the fp64 tolerances.
__device__ __forceinline__ double inv_sqrt(double x) {
  double y = __builtin_amdgcn_rsq(x);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const double e = fma(-x * y, y, 1.0);  // 1 - x y^2
    y = fma(0.5 * y, e, y);
  }
  return y;
}

// spline5 switch sw(r) and its derivative over the window [rs, rc)
__device__ __forceinline__ double switch5(double r, double rs, double rc, double inv_sw,
                                          double* dsw) {
  if (r < rs) {
    *dsw = 0.0;
    return 1.0;
  }
  if (r >= rc) {
    *dsw = 0.0;
    return 0.0;
  }
  const double u = (r - rs) * inv_sw;
  const double u2 = u * u, u3 = u2 * u;
  *dsw = (3.0 * u2 * (-6.0 * u2 + 15.0 * u - 10.0) + u3 * (-12.0 * u + 15.0)) * inv_sw;
  return u3 * (-6.0 * u2 + 15.0 * u - 10.0) + 1.0;
}

// The normalised env row [sw/r, sw x/r^2, sw y/r^2, sw z/r^2] of one slot.
__device__ __forceinline__ void env_value(double d0, double d1, double d2, double rs, double rc,
                                          double inv_sw, const double* avg, const double* isd,
                                          double* Rn) {
  const double r2 = d0 * d0 + d1 * d1 + d2 * d2;
  const double inv_r = inv_sqrt(r2);
  const double r = r2 * inv_r;
  double sw;
  if (r < rs) {
    sw = 1.0;
  } else if (r >= rc) {
    sw = 0.0;
  } else {
    const double u = (r - rs) * inv_sw;
    const double u2 = u * u, u3 = u2 * u;
    sw = u3 * (-6.0 * u2 + 15.0 * u - 10.0) + 1.0;
  }
  const double q = sw * inv_r * inv_r;
  Rn[0] = (sw * inv_r - avg[0]) * isd[0];
  Rn[1] = (q * d0 - avg[1]) * isd[1];
  Rn[2] = (q * d1 - avg[2]) * isd[2];
  Rn[3] = (q * d2 - avg[3]) * isd[3];
}

// Edge gradient g = sum_m nd[m] * d(Rn_m)/dd for one slot.
__device__ __forceinline__ void env_grad(double d0, double d1, double d2, double rs, double rc,
                                         double inv_sw, const double* isd, const double* nd,
                                         double* gv) {
  const double d[3] = {d0, d1, d2};
  const double r2 = d0 * d0 + d1 * d1 + d2 * d2;
  const double inv_r = inv_sqrt(r2);
  const double r = r2 * inv_r;
  double dsw;
  const double sw = switch5(r, rs, rc, inv_sw, &dsw);
  const double inv_r2 = inv_r * inv_r;
  const double dR0_dr = dsw * inv_r - sw * inv_r2;
  const double q = sw * inv_r2;
  const double dq_dr = dsw * inv_r2 - 2.0 * sw * inv_r2 * inv_r;
  const double w0 = nd[0] * isd[0];
  const double w[3] = {nd[1] * isd[1], nd[2] * isd[2], nd[3] * isd[3]};
  // sum_c w_c d_c, used by the radial part of R_1..3
  const double wd = w[0] * d[0] + w[1] * d[1] + w[2] * d[2];
#pragma unroll
  for (int mm = 0; mm < 3; ++mm) {
    const double ur = d[mm] * inv_r;
    gv[mm] = w0 * dR0_dr * ur + w[mm] * q + wd * dq_dr * ur;
  }
}

// One slot's outputs. The centre side (force += g, frame virial -= g (x) d)
// goes into the slot lane's LDS cells own[12], each cell added in tile order
// by one lane; the neighbour side (force -= g and, when asked for, the atom
// virial -= g (x) d, charged to the neighbour as in
// deepmd-op/overlays/op/pt/edge_force_virial.cu:138-146) is scattered in
// fixed point onto atom j. g = dE/d(x_j - x_i), d = x_j - x_i.
//   AV false (no atom virials): lane group 0 of the slot's column alone
//     (three atomics per slot).
//   AV true: all four lane groups grp (each holds the slot's g, d and j),
//     three of the twelve values each: group 0 the force, group 1 + c row c
//     of the virial, so that a wave instruction carries the atomics of 64
//     lanes instead of 16 (Cu-131k with atom virials: 29.2 -> 28.2 ms per
//     step). The kernels are instantiated for both: forming the edge
//     gradient on all 64 lanes, or the branch for both forms in one kernel,
//     cost the water backward 2-4 % without atom virials.
// g itself is stored (group 0) only when the caller keeps edge gradients.
template <bool AV>
__device__ __forceinline__ void edge_out(const EmbArgs& a, long e, int t, const double d[3],
                                         const double gv[3], double* own, int grp) {
  if (grp == 0) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      __hip_atomic_fetch_add(own + c, gv[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
      if constexpr (!AV) {
#pragma unroll
        for (int q = 0; q < 3; ++q)
          __hip_atomic_fetch_add(own + 3 + 3 * c + q, -gv[c] * d[q], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WAVEFRONT);
      }
    }
    // range guard of the fixed point: a NaN or an out-of-range gradient
    // would wrap silently in the integer sums
    const double gm = fmax(fabs(gv[0]), fmax(fabs(gv[1]), fabs(gv[2])));
    if (!(gm <= a.fix_gmax)) atomicOr(a.status, kStatusFixedRange);
    unsigned long long* fa = a.facc + 3L * t;
    fixed_add(fa, gv[0]);
    fixed_add(fa + 1, gv[1]);
    fixed_add(fa + 2, gv[2]);
    if (a.edge_grad) {
      double* eg = a.edge_grad + e * 3;
      eg[0] = gv[0];
      eg[1] = gv[1];
      eg[2] = gv[2];
    }
  } else if constexpr (AV) {
    const int c = grp - 1;
    const double gc = grp == 1 ? gv[0] : grp == 2 ? gv[1] : gv[2];
    unsigned long long* va = a.vacc + 9L * t + 3 * c;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const double v = -gc * d[q];
      __hip_atomic_fetch_add(own + 3 + 3 * c + q, v, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WAVEFRONT);
      fixed_add(va + q, v);
    }
  }
}

// End of an item (centre i, section tj): sums the 16 slot lanes' cells in a
// fixed order into cpsec[i][tj][12] and clears them for the next item; zeroes
// the kept edge gradients of the section's padded slots.
__device__ __forceinline__ void own_flush(const EmbArgs& a, int i, int tj, int nr, long ebase,
                                         double* own_w, int lane) {
  wave_lds_sync();
  if (lane < 12) {
    double s = 0.0;
    for (int k = 0; k < 16; ++k) s += own_w[12 * k + lane];
    a.cpsec[((long)i * a.ntypes + tj) * 12 + lane] = s;
  }
  wave_lds_sync();
  for (int q = lane; q < 16 * 12; q += 64) own_w[q] = 0.0;
  wave_lds_sync();
  if (a.edge_grad) {
    for (int sl = nr + lane; sl < a.sel[tj]; sl += 64) {
      double* eg = a.edge_grad + (ebase + sl) * 3;
      eg[0] = 0.0;
      eg[1] = 0.0;
      eg[2] = 0.0;
    }
  }
}

// The backward's fixed-point sums set to zero, spread over the forward's
// whole grid and issued as each block ends (no load of the block waits
// behind these stores), so the step needs no clearing kernel of its own.
__device__ __forceinline__ void clear_fixed(const EmbArgs& a) {
  const long n = a.zero_count ? (long)*a.zero_count : a.zero_n;
  const long stride = (long)gridDim.x * blockDim.x;
  const long q0 = (long)blockIdx.x * blockDim.x + threadIdx.x;
  for (long q = q0; q < 3 * n; q += stride) a.facc[q] = 0ull;
  if (a.vacc)
    for (long q = q0; q < 9 * n; q += stride) a.vacc[q] = 0ull;
}

__device__ __forceinline__ int find_pair(const EmbArgs& a) {
  int p = 0;
  while (p + 1 < a.npair && (int)blockIdx.x >= a.block_off[p + 1]) ++p;
  return p;
}

}  // namespace dpamd
