/*
 * TEST INFRASTRUCTURE ONLY — network half of the CPU oracle: environment
 * matrix, embedding nets, descriptor, fitting net, hand-written reverse-mode
 * backward and ProdForce / ProdVirial, fp64 throughout, OpenMP over centres.
 *
 * Semantics (DeepPot-SE se_e2_a; upstream DeePMD-kit 46fdc3e8 is absent, so
 * each convention is fixed here and restated in the GPU library):
 *  - switch (spline5): u = (r-rs)/(rc-rs); sw = 1 (r<rs),
 *    u^3(-6u^2+15u-10)+1 (rs<=r<rc), 0 (r>=rc);
 *  - env row [sw/r, sw*x/r^2, sw*y/r^2, sw*z/r^2] with (x,y,z) = x_j - x_i,
 *    padded rows 0, then (row - davg[ti][tj]) / dstd[ti][tj];
 *  - embedding net per (ti, tj): s -> L1 -> L2 -> L3, tanh; out == in gives
 *    y = x + tanh(xW+b), out == 2*in gives y = [x,x] + tanh(xW+b);
 *  - T = (1/nnei) sum_slots R^T G (padded slots included, G at s_pad),
 *    D[a][b] = sum_k T[k][a] T[k][b], b < axis, flattened a*axis + b;
 *  - fitting net per centre type: tanh hidden layers, y = x + idt*tanh(xW+b)
 *    when out == in, linear head, E_i = head + bias_atom_e[ti]
 *    (reference fitting semantics: deepmd-op/overlays/op/pt/graph_fitting.cu:1-25);
 *  - edge gradient g = dE/d(x_j - x_i); F_i += g, F_j -= g;
 *    atom_virial[j][3c+d] += -g_c * (x_j - x_i)_d (source-charged, reference
 *    deepmd-op/overlays/op/pt/edge_force_virial.cu:1-14, :138-146).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "se_e2_a.h"

long orc_emb_block_size(const orc_model* m) {
  const int L1 = m->emb[0], L2 = m->emb[1], L3 = m->emb[2];
  return (long)L1 + L1 + (long)L1 * L2 + L2 + (long)L2 * L3 + L3;
}

static int fit_in(const orc_model* m, int k) {
  return k == 0 ? m->emb[2] * m->axis : m->fit[k - 1];
}

long orc_fit_block_size(const orc_model* m) {
  long n = 0;
  for (int k = 0; k < 3; ++k) {
    const int in = fit_in(m, k), out = m->fit[k];
    n += (long)in * out + out + (out == in ? out : 0);
  }
  return n + m->fit[2] + 1;
}

double orc_switch(double r, double rs, double rc, double* dsw) {
  if (r < rs) {
    *dsw = 0.0;
    return 1.0;
  }
  if (r >= rc) {
    *dsw = 0.0;
    return 0.0;
  }
  const double u = (r - rs) / (rc - rs);
  const double u2 = u * u, u3 = u2 * u;
  *dsw = (3.0 * u2 * (-6.0 * u2 + 15.0 * u - 10.0) + u3 * (-12.0 * u + 15.0)) / (rc - rs);
  return u3 * (-6.0 * u2 + 15.0 * u - 10.0) + 1.0;
}

/* One slot's raw env row and its derivative w.r.t. d = x_j - x_i. */
static void env_row(const orc_model* m, const double* d, double R[4], double dR[4][3]) {
  const double r2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
  const double r = sqrt(r2);
  double dsw;
  const double sw = orc_switch(r, m->rcut_smth, m->rcut, &dsw);
  const double inv_r = 1.0 / r;
  const double inv_r2 = inv_r * inv_r;
  R[0] = sw * inv_r;
  for (int c = 0; c < 3; ++c) R[1 + c] = sw * d[c] * inv_r2;
  const double dR0_dr = dsw * inv_r - sw * inv_r2;
  const double dq_dr = dsw * inv_r2 - 2.0 * sw * inv_r2 * inv_r; /* q = sw / r^2 */
  const double q = sw * inv_r2;
  for (int mm = 0; mm < 3; ++mm) {
    const double ur = d[mm] * inv_r; /* dr/dd_m */
    dR[0][mm] = dR0_dr * ur;
    for (int c = 0; c < 3; ++c) dR[1 + c][mm] = (c == mm ? q : 0.0) + d[c] * dq_dr * ur;
  }
}

void orc_env_mat(const orc_model* m, int nloc, const double* ext, const int* type,
                 const int* nlist, double* env, double* env_deriv, double* rij) {
  for (int i = 0; i < nloc; ++i) {
    const int ti = type[i] < 0 ? 0 : type[i];
    for (int t = 0; t < m->ntypes; ++t) {
      const double* avg = m->davg + ((long)ti * m->ntypes + t) * 4;
      const double* std = m->dstd + ((long)ti * m->ntypes + t) * 4;
      for (int s = m->sec[t]; s < m->sec[t + 1]; ++s) {
        const long e = (long)i * m->nnei + s;
        const int j = nlist[e];
        double R[4] = {0, 0, 0, 0}, dR[4][3] = {{0}}, d[3] = {0, 0, 0};
        if (j >= 0) {
          for (int c = 0; c < 3; ++c) d[c] = ext[3L * j + c] - ext[3L * i + c];
          env_row(m, d, R, dR);
        }
        for (int k = 0; k < 4; ++k) {
          if (env) env[e * 4 + k] = (R[k] - avg[k]) / std[k];
          if (env_deriv)
            for (int c = 0; c < 3; ++c) env_deriv[(e * 4 + k) * 3 + c] = dR[k][c] / std[k];
        }
        if (rij)
          for (int c = 0; c < 3; ++c) rij[e * 3 + c] = d[c];
      }
    }
  }
}

/* y = act(x W + b) with the residual rule; t keeps tanh(xW+b) for backward. */
static void emb_layer(const double* x, int in, const double* W, const double* b, int out,
                      double* y, double* t) {
  for (int f = 0; f < out; ++f) {
    double z = 0.0;
    for (int k = 0; k < in; ++k) z += x[k] * W[(long)k * out + f];
    t[f] = tanh(z + b[f]);
  }
  for (int f = 0; f < out; ++f) {
    double res = 0.0;
    if (out == in) res = x[f];
    else if (out == 2 * in) res = x[f % in];
    y[f] = res + t[f];
  }
}

static void emb_forward(const orc_model* m, const double* P, double s, double* y1, double* t1,
                        double* y2, double* t2, double* y3, double* t3) {
  const int L1 = m->emb[0], L2 = m->emb[1], L3 = m->emb[2];
  const double* W1 = P;
  const double* b1 = W1 + L1;
  const double* W2 = b1 + L1;
  const double* b2 = W2 + (long)L1 * L2;
  const double* W3 = b2 + L2;
  const double* b3 = W3 + (long)L2 * L3;
  emb_layer(&s, 1, W1, b1, L1, y1, t1);
  emb_layer(y1, L1, W2, b2, L2, y2, t2);
  emb_layer(y2, L2, W3, b3, L3, y3, t3);
}

/* dx = reverse of emb_layer given dy; also uses t = tanh part. */
static void emb_layer_back(const double* dy, int in, const double* W, int out, const double* t,
                           double* dz, double* dx) {
  for (int f = 0; f < out; ++f) dz[f] = dy[f] * (1.0 - t[f] * t[f]);
  for (int k = 0; k < in; ++k) {
    double acc = 0.0;
    for (int f = 0; f < out; ++f) acc += dz[f] * W[(long)k * out + f];
    if (out == in) acc += dy[k];
    else if (out == 2 * in) acc += dy[k] + dy[k + in];
    dx[k] = acc;
  }
}

void orc_embed(const orc_model* m, int ti, int tj, double s, double* g) {
  const int L1 = m->emb[0], L2 = m->emb[1], L3 = m->emb[2];
  const double* P = m->emb_params + ((long)ti * m->ntypes + tj) * orc_emb_block_size(m);
  double* buf = (double*)malloc(sizeof(double) * (size_t)(2 * (L1 + L2 + L3)));
  emb_forward(m, P, s, buf, buf + L1, buf + 2 * L1, buf + 2 * L1 + L2, g, buf + 2 * (L1 + L2));
  free(buf);
}

typedef struct {
  double *env, *envd, *d;            /* nnei*4, nnei*12, nnei*3 */
  double *y1, *t1, *y2, *t2, *G, *t3; /* per slot activations */
  double *T, *dT, *D, *dD;
  double *h[3], *th[3], *dh, *dz, *dx;
  double *dG, *dy2, *dz3, *dy1, *dz2, *dz1;
} scratch;

static void* xcalloc(size_t n, size_t sz) { return calloc(n ? n : 1, sz); }

static void scratch_alloc(const orc_model* m, scratch* s) {
  const int nnei = m->nnei, L1 = m->emb[0], L2 = m->emb[1], L3 = m->emb[2];
  const int Dn = L3 * m->axis;
  int maxw = Dn;
  for (int k = 0; k < 3; ++k)
    if (m->fit[k] > maxw) maxw = m->fit[k];
  s->env = xcalloc((size_t)nnei * 4, 8);
  s->envd = xcalloc((size_t)nnei * 12, 8);
  s->d = xcalloc((size_t)nnei * 3, 8);
  s->y1 = xcalloc((size_t)nnei * L1, 8);
  s->t1 = xcalloc((size_t)nnei * L1, 8);
  s->y2 = xcalloc((size_t)nnei * L2, 8);
  s->t2 = xcalloc((size_t)nnei * L2, 8);
  s->G = xcalloc((size_t)nnei * L3, 8);
  s->t3 = xcalloc((size_t)nnei * L3, 8);
  s->T = xcalloc((size_t)4 * L3, 8);
  s->dT = xcalloc((size_t)4 * L3, 8);
  s->D = xcalloc((size_t)Dn, 8);
  s->dD = xcalloc((size_t)Dn, 8);
  for (int k = 0; k < 3; ++k) {
    s->h[k] = xcalloc((size_t)m->fit[k], 8);
    s->th[k] = xcalloc((size_t)m->fit[k], 8);
  }
  s->dh = xcalloc((size_t)maxw, 8);
  s->dz = xcalloc((size_t)maxw, 8);
  s->dx = xcalloc((size_t)maxw, 8);
  s->dG = xcalloc((size_t)L3, 8);
  s->dy2 = xcalloc((size_t)L2, 8);
  s->dz3 = xcalloc((size_t)L3, 8);
  s->dy1 = xcalloc((size_t)L1, 8);
  s->dz2 = xcalloc((size_t)L2, 8);
  s->dz1 = xcalloc((size_t)L1, 8);
}

static void scratch_free(scratch* s) {
  free(s->env); free(s->envd); free(s->d);
  free(s->y1); free(s->t1); free(s->y2); free(s->t2); free(s->G); free(s->t3);
  free(s->T); free(s->dT); free(s->D); free(s->dD);
  for (int k = 0; k < 3; ++k) { free(s->h[k]); free(s->th[k]); }
  free(s->dh); free(s->dz); free(s->dx);
  free(s->dG); free(s->dy2); free(s->dz3); free(s->dy1); free(s->dz2); free(s->dz1);
}

/* Fitting forward + input gradient for one centre; returns the atomic energy. */
static double fitting(const orc_model* m, int ti, scratch* s) {
  const double* P = m->fit_params + (long)ti * orc_fit_block_size(m);
  const double* W[3];
  const double* b[3];
  const double* idt[3];
  const double* p = P;
  for (int k = 0; k < 3; ++k) {
    const int in = fit_in(m, k), out = m->fit[k];
    W[k] = p; p += (long)in * out;
    b[k] = p; p += out;
    idt[k] = (out == in) ? p : NULL;
    if (out == in) p += out;
  }
  const double* Wo = p;
  const double bo = p[m->fit[2]];
  const double* x = s->D;
  for (int k = 0; k < 3; ++k) {
    const int in = fit_in(m, k), out = m->fit[k];
    double* z = s->dz; /* reuse as temporary */
    for (int f = 0; f < out; ++f) z[f] = 0.0;
    for (int q = 0; q < in; ++q) {
      const double xq = x[q];
      const double* w = W[k] + (long)q * out;
      for (int f = 0; f < out; ++f) z[f] += xq * w[f];
    }
    for (int f = 0; f < out; ++f) {
      s->th[k][f] = tanh(z[f] + b[k][f]);
      s->h[k][f] = idt[k] ? x[f] + idt[k][f] * s->th[k][f] : s->th[k][f];
    }
    x = s->h[k];
  }
  double e = 0.0;
  for (int f = 0; f < m->fit[2]; ++f) e += x[f] * Wo[f];
  e += bo + m->bias_atom_e[ti];
  /* backward */
  double* dh = s->dh;
  for (int f = 0; f < m->fit[2]; ++f) dh[f] = Wo[f];
  for (int k = 2; k >= 0; --k) {
    const int in = fit_in(m, k), out = m->fit[k];
    double* dz = s->dz;
    for (int f = 0; f < out; ++f) {
      const double g = 1.0 - s->th[k][f] * s->th[k][f];
      dz[f] = dh[f] * (idt[k] ? idt[k][f] : 1.0) * g;
    }
    double* dx = (k == 0) ? s->dD : s->dx;
    for (int q = 0; q < in; ++q) {
      const double* w = W[k] + (long)q * out;
      double acc = 0.0;
      for (int f = 0; f < out; ++f) acc += dz[f] * w[f];
      dx[q] = acc + (idt[k] ? dh[q] : 0.0);
    }
    if (k > 0) memcpy(dh, dx, sizeof(double) * (size_t)in);
  }
  return e;
}

static void eval_centre(const orc_model* m, int i, const double* ext, const int* type,
                        const int* nlist, scratch* s, double* atom_energy, double* descrpt,
                        double* dE_dD, double* net_deriv, double* edge_grad) {
  const int nnei = m->nnei, L1 = m->emb[0], L2 = m->emb[1], L3 = m->emb[2], M2 = m->axis;
  const long eb = orc_emb_block_size(m);
  const int ti = type[i];
  double* eg = edge_grad + (long)i * nnei * 3;
  if (ti < 0) {
    atom_energy[i] = 0.0;
    memset(eg, 0, sizeof(double) * (size_t)nnei * 3);
    if (descrpt) memset(descrpt + (long)i * L3 * M2, 0, sizeof(double) * (size_t)L3 * M2);
    if (dE_dD) memset(dE_dD + (long)i * L3 * M2, 0, sizeof(double) * (size_t)L3 * M2);
    if (net_deriv) memset(net_deriv + (long)i * nnei * 4, 0, sizeof(double) * (size_t)nnei * 4);
    return;
  }
  /* env mat + embedding forward for every slot (padded slots included) */
  for (int t = 0; t < m->ntypes; ++t) {
    const double* avg = m->davg + ((long)ti * m->ntypes + t) * 4;
    const double* std = m->dstd + ((long)ti * m->ntypes + t) * 4;
    const double* P = m->emb_params + ((long)ti * m->ntypes + t) * eb;
    for (int sl = m->sec[t]; sl < m->sec[t + 1]; ++sl) {
      const int j = nlist[(long)i * nnei + sl];
      double R[4] = {0, 0, 0, 0}, dR[4][3] = {{0}};
      double* d = s->d + 3 * sl;
      d[0] = d[1] = d[2] = 0.0;
      if (j >= 0) {
        for (int c = 0; c < 3; ++c) d[c] = ext[3L * j + c] - ext[3L * i + c];
        env_row(m, d, R, dR);
      }
      for (int k = 0; k < 4; ++k) {
        s->env[sl * 4 + k] = (R[k] - avg[k]) / std[k];
        for (int c = 0; c < 3; ++c) s->envd[(sl * 4 + k) * 3 + c] = dR[k][c] / std[k];
      }
      emb_forward(m, P, s->env[sl * 4], s->y1 + (long)sl * L1, s->t1 + (long)sl * L1,
                  s->y2 + (long)sl * L2, s->t2 + (long)sl * L2, s->G + (long)sl * L3,
                  s->t3 + (long)sl * L3);
    }
  }
  /* T = (1/nnei) sum R^T G */
  const double inv_n = 1.0 / (double)nnei;
  for (int q = 0; q < 4 * L3; ++q) s->T[q] = 0.0;
  for (int sl = 0; sl < nnei; ++sl)
    for (int k = 0; k < 4; ++k) {
      const double r = s->env[sl * 4 + k];
      const double* g = s->G + (long)sl * L3;
      double* Tk = s->T + k * L3;
      for (int a = 0; a < L3; ++a) Tk[a] += r * g[a];
    }
  for (int q = 0; q < 4 * L3; ++q) s->T[q] *= inv_n;
  /* D = T^T T[:, :M2] */
  for (int a = 0; a < L3; ++a)
    for (int b = 0; b < M2; ++b) {
      double acc = 0.0;
      for (int k = 0; k < 4; ++k) acc += s->T[k * L3 + a] * s->T[k * L3 + b];
      s->D[a * M2 + b] = acc;
    }
  if (descrpt) memcpy(descrpt + (long)i * L3 * M2, s->D, sizeof(double) * (size_t)L3 * M2);
  atom_energy[i] = fitting(m, ti, s);
  if (dE_dD) memcpy(dE_dD + (long)i * L3 * M2, s->dD, sizeof(double) * (size_t)L3 * M2);
  /* dT */
  for (int k = 0; k < 4; ++k)
    for (int a = 0; a < L3; ++a) {
      double acc = 0.0;
      for (int b = 0; b < M2; ++b) acc += s->dD[a * M2 + b] * s->T[k * L3 + b];
      if (a < M2)
        for (int a2 = 0; a2 < L3; ++a2) acc += s->dD[a2 * M2 + a] * s->T[k * L3 + a2];
      s->dT[k * L3 + a] = acc;
    }
  /* per slot: dR_norm, dG, embedding backward, edge gradient */
  for (int t = 0; t < m->ntypes; ++t) {
    const double* P = m->emb_params + ((long)ti * m->ntypes + t) * eb;
    const double* W1 = P;
    const double* W2 = W1 + 2 * L1;
    const double* W3 = W2 + (long)L1 * L2 + L2;
    for (int sl = m->sec[t]; sl < m->sec[t + 1]; ++sl) {
      const double* g = s->G + (long)sl * L3;
      const double* R = s->env + sl * 4;
      double nd[4];
      for (int k = 0; k < 4; ++k) {
        double acc = 0.0;
        for (int a = 0; a < L3; ++a) acc += g[a] * s->dT[k * L3 + a];
        nd[k] = acc * inv_n;
      }
      for (int a = 0; a < L3; ++a) {
        double acc = 0.0;
        for (int k = 0; k < 4; ++k) acc += R[k] * s->dT[k * L3 + a];
        s->dG[a] = acc * inv_n;
      }
      emb_layer_back(s->dG, L2, W3, L3, s->t3 + (long)sl * L3, s->dz3, s->dy2);
      emb_layer_back(s->dy2, L1, W2, L2, s->t2 + (long)sl * L2, s->dz2, s->dy1);
      double ds;
      emb_layer_back(s->dy1, 1, W1, L1, s->t1 + (long)sl * L1, s->dz1, &ds);
      nd[0] += ds;
      if (net_deriv)
        for (int k = 0; k < 4; ++k) net_deriv[((long)i * nnei + sl) * 4 + k] = nd[k];
      const int j = nlist[(long)i * nnei + sl];
      for (int c = 0; c < 3; ++c) {
        double acc = 0.0;
        if (j >= 0)
          for (int k = 0; k < 4; ++k) acc += nd[k] * s->envd[(sl * 4 + k) * 3 + c];
        eg[sl * 3 + c] = acc;
      }
    }
  }
}

/*
 * Full evaluation on an extended system: centres 0..nloc-1, neighbours index
 * the nall extended atoms. force / atom_virial are over the nall atoms (ghost
 * contributions stay in ghost slots, as the LAMMPS pair path expects,
 * pair_deepmd.cpp:603-608). Optional outputs may be NULL.
 */
int orc_eval(const orc_model* m, int nloc, int nall, const double* ext, const int* type,
             const int* nlist, int nthreads, double* atom_energy, double* descrpt, double* dE_dD,
             double* net_deriv, double* edge_grad, double* force, double* virial,
             double* atom_virial) {
  const int nnei = m->nnei;
  double* eg = edge_grad;
  if (!eg) eg = (double*)malloc(sizeof(double) * 3 * (size_t)(nloc > 0 ? nloc : 1) * nnei);
  if (!eg) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    scratch s;
    scratch_alloc(m, &s);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
    for (int i = 0; i < nloc; ++i)
      eval_centre(m, i, ext, type, nlist, &s, atom_energy, descrpt, dE_dD, net_deriv, eg);
    scratch_free(&s);
  }
  (void)nthreads;
  orc_prod_force(nloc, nall, nnei, ext, nlist, eg, force, virial, atom_virial);
  if (!edge_grad) free(eg);
  return 0;
}

/*
 * ProdForce / ProdVirial from per-slot edge gradients g = dE/d(x_j - x_i),
 * summed in (centre, slot) order: F_i += g, F_j -= g, W[3c+d] -= g_c d_d with
 * d = x_j - x_i, the per-atom share charged to the neighbour j
 * (edge_force_virial.cu:1-14, :138-146 of the reference). Over the nall
 * extended atoms; ghost contributions stay in ghost slots (orc_fold moves
 * them onto owners). Slots with nlist < 0 are skipped.
 */
void orc_prod_force(int nloc, int nall, int nnei, const double* ext, const int* nlist,
                    const double* edge_grad, double* force, double* virial,
                    double* atom_virial) {
  memset(force, 0, sizeof(double) * 3 * (size_t)nall);
  memset(virial, 0, sizeof(double) * 9);
  if (atom_virial) memset(atom_virial, 0, sizeof(double) * 9 * (size_t)nall);
  for (int i = 0; i < nloc; ++i)
    for (int sl = 0; sl < nnei; ++sl) {
      const int j = nlist[(long)i * nnei + sl];
      if (j < 0) continue;
      const double* g = edge_grad + ((long)i * nnei + sl) * 3;
      double d[3];
      for (int c = 0; c < 3; ++c) d[c] = ext[3L * j + c] - ext[3L * i + c];
      for (int c = 0; c < 3; ++c) {
        force[3L * i + c] += g[c];
        force[3L * j + c] -= g[c];
      }
      for (int c = 0; c < 3; ++c)
        for (int dd = 0; dd < 3; ++dd) {
          const double v = -g[c] * d[dd];
          virial[3 * c + dd] += v;
          if (atom_virial) atom_virial[9L * j + 3 * c + dd] += v;
        }
    }
}

/* Fold ghost-image force / atom virial onto their owners (standalone path). */
void orc_fold(int nloc, int nall, const int* mapping, const double* force_ext,
              const double* atom_virial_ext, double* force, double* atom_virial) {
  memset(force, 0, sizeof(double) * 3 * (size_t)nloc);
  if (atom_virial) memset(atom_virial, 0, sizeof(double) * 9 * (size_t)nloc);
  for (int j = 0; j < nall; ++j) {
    const int o = mapping[j];
    for (int c = 0; c < 3; ++c) force[3L * o + c] += force_ext[3L * j + c];
    if (atom_virial && atom_virial_ext)
      for (int c = 0; c < 9; ++c) atom_virial[9L * o + c] += atom_virial_ext[9L * j + c];
  }
}
