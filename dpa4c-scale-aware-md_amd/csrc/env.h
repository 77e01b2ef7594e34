// Environment row of one neighbour slot and its gradient, in fp64 (both
// precision modes compute the env matrix, the edge gradient and everything
// downstream of it in fp64), plus the (ti, tj) pair lookup of the embedding
// kernels' block table.
#pragma once

#include "kernels.h"

namespace dpamd {

// spline5 switch and the normalised env row [sw/r, sw x/r^2, sw y/r^2, sw z/r^2].
__device__ __forceinline__ void env_value(double d0, double d1, double d2, double rs, double rc,
                                          const double* avg, const double* sd, double* Rn) {
  const double r2 = d0 * d0 + d1 * d1 + d2 * d2;
  const double r = sqrt(r2);
  double sw;
  if (r < rs) {
    sw = 1.0;
  } else if (r >= rc) {
    sw = 0.0;
  } else {
    const double u = (r - rs) / (rc - rs);
    const double u2 = u * u, u3 = u2 * u;
    sw = u3 * (-6.0 * u2 + 15.0 * u - 10.0) + 1.0;
  }
  const double inv_r = 1.0 / r;
  const double inv_r2 = inv_r * inv_r;
  Rn[0] = (sw * inv_r - avg[0]) / sd[0];
  Rn[1] = (sw * d0 * inv_r2 - avg[1]) / sd[1];
  Rn[2] = (sw * d1 * inv_r2 - avg[2]) / sd[2];
  Rn[3] = (sw * d2 * inv_r2 - avg[3]) / sd[3];
}

// Edge gradient g = sum_m nd[m] * d(Rn_m)/dd for one slot.
__device__ __forceinline__ void env_grad(double d0, double d1, double d2, double rs, double rc,
                                         const double* sd, const double* nd, double* gv) {
  const double d[3] = {d0, d1, d2};
  const double r2 = d0 * d0 + d1 * d1 + d2 * d2;
  const double r = sqrt(r2);
  double sw, dsw;
  if (r < rs) {
    sw = 1.0;
    dsw = 0.0;
  } else if (r >= rc) {
    sw = 0.0;
    dsw = 0.0;
  } else {
    const double u = (r - rs) / (rc - rs);
    const double u2 = u * u, u3 = u2 * u;
    sw = u3 * (-6.0 * u2 + 15.0 * u - 10.0) + 1.0;
    dsw = (3.0 * u2 * (-6.0 * u2 + 15.0 * u - 10.0) + u3 * (-12.0 * u + 15.0)) / (rc - rs);
  }
  const double inv_r = 1.0 / r;
  const double inv_r2 = inv_r * inv_r;
  const double dR0_dr = dsw * inv_r - sw * inv_r2;
  const double q = sw * inv_r2;
  const double dq_dr = dsw * inv_r2 - 2.0 * sw * inv_r2 * inv_r;
  const double w0 = nd[0] / sd[0];
  const double w[3] = {nd[1] / sd[1], nd[2] / sd[2], nd[3] / sd[3]};
  // sum_c w_c d_c, used by the radial part of R_1..3
  const double wd = w[0] * d[0] + w[1] * d[1] + w[2] * d[2];
#pragma unroll
  for (int mm = 0; mm < 3; ++mm) {
    const double ur = d[mm] * inv_r;
    gv[mm] = w0 * dR0_dr * ur + w[mm] * q + wd * dq_dr * ur;
  }
}

__device__ __forceinline__ int find_pair(const EmbArgs& a) {
  int p = 0;
  while (p + 1 < a.npair && (int)blockIdx.x >= a.block_off[p + 1]) ++p;
  return p;
}

}  // namespace dpamd
