/*
 * TEST INFRASTRUCTURE ONLY — geometry half of the CPU oracle (ghost images,
 * candidate neighbour lists, per-type sel formatting). Compiled with
 * -ffp-contract=off so that every distance is the plain IEEE sequence
 *   dx = xj - xi; r2 = dx*dx + dy*dy + dz*dz
 * which the GPU path reproduces bit for bit; the neighbour list is then
 * bit-exact by construction and the tests check it is.
 *
 * Conventions fixed here (upstream DeePMD-kit is not vendored, so these are
 * this oracle's definitions, documented next to each function):
 *  - box is LAMMPS' row-major h = [xx,0,0, xy,yy,0, xz,yz,zz]
 *    (lammps-deepmd-plugin/src/pair_deepmd.cpp:293-299);
 *  - neighbours are kept when r2 <= rcut*rcut and sorted by the key
 *    (type_j, r2, j); section t holds the first sel[t] of type t, padded -1
 *    (DeepPot-SE neighbour formatting; reference analog: the exact-cut predicate
 *    production/dpa4c-runtime/include/dpa_chain/exact_cut.cuh:10-20).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "se_e2_a.h"

/* Perpendicular heights of the cell and the cutoff in fractional units. */
static int box_geometry(const double* box, double rcut, double rcf[3], int nrep[3]) {
  const double xx = box[0], xy = box[3], yy = box[4], xz = box[6], yz = box[7], zz = box[8];
  if (box[1] != 0.0 || box[2] != 0.0 || box[5] != 0.0) return -1;
  if (!(xx > 0.0 && yy > 0.0 && zz > 0.0)) return -1;
  const double vol = xx * yy * zz;
  const double bc0 = yy * zz, bc1 = xy * zz, bc2 = xy * yz - yy * xz;
  const double ha = vol / sqrt(bc0 * bc0 + bc1 * bc1 + bc2 * bc2);
  const double hb = (yy * zz) / sqrt(zz * zz + yz * yz);
  const double hc = zz;
  rcf[0] = rcut / ha;
  rcf[1] = rcut / hb;
  rcf[2] = rcut / hc;
  for (int d = 0; d < 3; ++d) nrep[d] = (int)ceil(rcf[d]);
  return 0;
}

static void to_frac(const double* box, const double* x, double* s) {
  s[2] = x[2] / box[8];
  s[1] = (x[1] - s[2] * box[7]) / box[4];
  s[0] = (x[0] - s[1] * box[3] - s[2] * box[6]) / box[0];
}

static void wrap(const double* box, const double* x, double* xw, double* sw) {
  double s[3];
  to_frac(box, x, s);
  const double n0 = floor(s[0]), n1 = floor(s[1]), n2 = floor(s[2]);
  xw[0] = x[0] - n0 * box[0] - n1 * box[3] - n2 * box[6];
  xw[1] = x[1] - n1 * box[4] - n2 * box[7];
  xw[2] = x[2] - n2 * box[8];
  to_frac(box, xw, sw);
}

/*
 * Ghost images: local atoms are wrapped into the cell first; then for every
 * shift (nc outer, nb, na inner; the zero shift skipped) and every atom k in
 * order, the image x_k + na*a + nb*b + nc*c is kept when each fractional
 * coordinate s_d + n_d lies in [-rcf_d, 1 + rcf_d). Ghost index = nloc +
 * running count, mapping[ghost] = k. Reference analog of the standalone path:
 * copy_coord in DeepPotPTExpt.cc:1737-1745.
 */
static int ghosts_impl(int nloc, const double* coord, const int* atype, const double* box,
                       double rcut, int cap, double* ext, int* ext_type, int* mapping) {
  double rcf[3];
  int nrep[3];
  if (box_geometry(box, rcut, rcf, nrep)) return -1;
  const double hi0 = 1.0 + rcf[0], hi1 = 1.0 + rcf[1], hi2 = 1.0 + rcf[2];
  double* xw = (double*)malloc(sizeof(double) * 3 * (size_t)(nloc > 0 ? nloc : 1));
  double* sw = (double*)malloc(sizeof(double) * 3 * (size_t)(nloc > 0 ? nloc : 1));
  for (int k = 0; k < nloc; ++k) wrap(box, coord + 3 * k, xw + 3 * k, sw + 3 * k);
  int n = 0;
  for (int k = 0; k < nloc; ++k, ++n) {
    if (ext && n < cap) {
      memcpy(ext + 3 * n, xw + 3 * k, 3 * sizeof(double));
      ext_type[n] = atype[k];
      mapping[n] = k;
    }
  }
  for (int nc = -nrep[2]; nc <= nrep[2]; ++nc)
    for (int nb = -nrep[1]; nb <= nrep[1]; ++nb)
      for (int na = -nrep[0]; na <= nrep[0]; ++na) {
        if (na == 0 && nb == 0 && nc == 0) continue;
        for (int k = 0; k < nloc; ++k) {
          const double f0 = sw[3 * k + 0] + (double)na;
          const double f1 = sw[3 * k + 1] + (double)nb;
          const double f2 = sw[3 * k + 2] + (double)nc;
          if (!(f0 >= -rcf[0] && f0 < hi0 && f1 >= -rcf[1] && f1 < hi1 && f2 >= -rcf[2] && f2 < hi2))
            continue;
          if (ext && n < cap) {
            const double* x = xw + 3 * k;
            ext[3 * n + 0] = x[0] + (double)na * box[0] + (double)nb * box[3] + (double)nc * box[6];
            ext[3 * n + 1] = x[1] + (double)nb * box[4] + (double)nc * box[7];
            ext[3 * n + 2] = x[2] + (double)nc * box[8];
            ext_type[n] = atype[k];
            mapping[n] = k;
          }
          ++n;
        }
      }
  free(xw);
  free(sw);
  return n;
}

int orc_ghost_count(int nloc, const double* coord, const double* box, double rcut) {
  return ghosts_impl(nloc, coord, NULL, box, rcut, 0, NULL, NULL, NULL);
}

int orc_build_ghosts(int nloc, const double* coord, const int* atype, const double* box,
                     double rcut, int nall_cap, double* ext_coord, int* ext_type, int* mapping) {
  const int n = ghosts_impl(nloc, coord, atype, box, rcut, nall_cap, ext_coord, ext_type, mapping);
  return (n > nall_cap) ? -2 : n;
}

static inline double dist2(const double* xi, const double* xj) {
  const double dx = xj[0] - xi[0];
  const double dy = xj[1] - xi[1];
  const double dz = xj[2] - xi[2];
  return dx * dx + dy * dy + dz * dz;
}

/* Brute force O(nloc*nall): all j != i (type >= 0) with r2 <= rc*rc, j ascending. */
long orc_candidates_brute(int nloc, int nall, const double* ext, const int* type, double rc,
                          long cap, long* offsets, int* cand) {
  const double rc2 = rc * rc;
  long n = 0;
  offsets[0] = 0;
  for (int i = 0; i < nloc; ++i) {
    if (type[i] >= 0) {
      for (int j = 0; j < nall; ++j) {
        if (j == i || type[j] < 0) continue;
        if (dist2(ext + 3 * i, ext + 3 * j) <= rc2) {
          if (n < cap) cand[n] = j;
          ++n;
        }
      }
    }
    offsets[i + 1] = n;
  }
  return n;
}

/*
 * Same set through Cartesian bins of edge >= rc over the bounding box of the
 * extended atoms (an independent method from the GPU's fractional cells).
 * Within a centre the output is sorted by j, so it equals the brute force.
 */
static int cmp_int(const void* a, const void* b) {
  const int x = *(const int*)a, y = *(const int*)b;
  return (x > y) - (x < y);
}

long orc_candidates_cell(int nloc, int nall, const double* ext, const int* type,
                         const double* box, double rc, long cap, long* offsets, int* cand) {
  (void)box;
  const double rc2 = rc * rc;
  double lo[3] = {1e300, 1e300, 1e300}, hi[3] = {-1e300, -1e300, -1e300};
  for (int j = 0; j < nall; ++j)
    for (int d = 0; d < 3; ++d) {
      if (ext[3 * j + d] < lo[d]) lo[d] = ext[3 * j + d];
      if (ext[3 * j + d] > hi[d]) hi[d] = ext[3 * j + d];
    }
  int nb[3];
  double bw[3];
  for (int d = 0; d < 3; ++d) {
    nb[d] = (int)floor((hi[d] - lo[d]) / (rc * 1.001));
    if (nb[d] < 1) nb[d] = 1;
    bw[d] = (hi[d] - lo[d]) / nb[d];
    if (bw[d] <= 0) bw[d] = 1.0;
  }
  const long nbins = (long)nb[0] * nb[1] * nb[2];
  int* bin_of = (int*)malloc(sizeof(int) * (size_t)(nall > 0 ? nall : 1));
  long* start = (long*)calloc((size_t)nbins + 1, sizeof(long));
  int* items = (int*)malloc(sizeof(int) * (size_t)(nall > 0 ? nall : 1));
  for (int j = 0; j < nall; ++j) {
    int c[3];
    for (int d = 0; d < 3; ++d) {
      c[d] = (int)floor((ext[3 * j + d] - lo[d]) / bw[d]);
      if (c[d] < 0) c[d] = 0;
      if (c[d] >= nb[d]) c[d] = nb[d] - 1;
    }
    bin_of[j] = (c[2] * nb[1] + c[1]) * nb[0] + c[0];
    start[bin_of[j] + 1]++;
  }
  for (long b = 0; b < nbins; ++b) start[b + 1] += start[b];
  long* fillp = (long*)malloc(sizeof(long) * (size_t)nbins);
  memcpy(fillp, start, sizeof(long) * (size_t)nbins);
  for (int j = 0; j < nall; ++j) items[fillp[bin_of[j]]++] = j;
  free(fillp);

  long n = 0;
  offsets[0] = 0;
  for (int i = 0; i < nloc; ++i) {
    const long first = n;
    if (type[i] >= 0) {
      const int b = bin_of[i];
      const int c0 = b % nb[0], c1 = (b / nb[0]) % nb[1], c2 = b / (nb[0] * nb[1]);
      for (int z = c2 - 1; z <= c2 + 1; ++z) {
        if (z < 0 || z >= nb[2]) continue;
        for (int y = c1 - 1; y <= c1 + 1; ++y) {
          if (y < 0 || y >= nb[1]) continue;
          for (int x = c0 - 1; x <= c0 + 1; ++x) {
            if (x < 0 || x >= nb[0]) continue;
            const int bb = (z * nb[1] + y) * nb[0] + x;
            for (long p = start[bb]; p < start[bb + 1]; ++p) {
              const int j = items[p];
              if (j == i || type[j] < 0) continue;
              if (dist2(ext + 3 * i, ext + 3 * j) <= rc2) {
                if (n < cap) cand[n] = j;
                ++n;
              }
            }
          }
        }
      }
      if (n <= cap) qsort(cand + first, (size_t)(n - first), sizeof(int), cmp_int);
    }
    offsets[i + 1] = n;
  }
  free(bin_of);
  free(start);
  free(items);
  return n;
}

typedef struct {
  int type;
  double r2;
  int j;
} nb_key;

static int cmp_key(const void* a, const void* b) {
  const nb_key* x = (const nb_key*)a;
  const nb_key* y = (const nb_key*)b;
  if (x->type != y->type) return x->type < y->type ? -1 : 1;
  if (x->r2 != y->r2) return x->r2 < y->r2 ? -1 : 1;
  return (x->j > y->j) - (x->j < y->j);
}

/*
 * sel formatting (upstream format_nlist, absent from the reference): keep
 * candidates with r2 <= rcut*rcut, sort by (type, r2, j), section t takes the
 * first sel[t] of type t, the rest of the section is -1.
 */
void orc_format_nlist(const orc_model* m, int nloc, const double* ext, const int* type,
                      const long* offsets, const int* cand, int* nlist) {
  const double rc2 = m->rcut * m->rcut;
  long maxc = 1;
  for (int i = 0; i < nloc; ++i)
    if (offsets[i + 1] - offsets[i] > maxc) maxc = offsets[i + 1] - offsets[i];
  nb_key* keys = (nb_key*)malloc(sizeof(nb_key) * (size_t)maxc);
  for (int i = 0; i < nloc; ++i) {
    int* row = nlist + (long)i * m->nnei;
    for (int s = 0; s < m->nnei; ++s) row[s] = -1;
    if (type[i] < 0) continue;
    int n = 0;
    for (long p = offsets[i]; p < offsets[i + 1]; ++p) {
      const int j = cand[p];
      if (j == i || type[j] < 0 || type[j] >= m->ntypes) continue;
      const double r2 = dist2(ext + 3 * (long)i, ext + 3 * (long)j);
      if (r2 <= rc2) {
        keys[n].type = type[j];
        keys[n].r2 = r2;
        keys[n].j = j;
        ++n;
      }
    }
    qsort(keys, (size_t)n, sizeof(nb_key), cmp_key);
    int fill[ORC_MAX_TYPES] = {0};
    for (int q = 0; q < n; ++q) {
      const int t = keys[q].type;
      if (fill[t] < m->sel[t]) row[m->sec[t] + fill[t]++] = keys[q].j;
    }
  }
  free(keys);
}
