/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle of this repository.
 *
 * A plain-C, fp64 restatement of the DeepPot-SE `se_e2_a` energy / force /
 * virial evaluation (neighbor list, sel formatting, environment matrix with
 * the spline5 switch, embedding nets, G^T R R^T G descriptor, fitting net,
 * hand-written reverse-mode backward, ProdForce / ProdVirial). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may call it, and
 * only as the checker. The shipped library never links it.
 *
 * The se_e2_a arithmetic lives in upstream DeePMD-kit (commit 46fdc3e8, pinned
 * in production/dpa4c-runtime/third_party/sources.lock.json:4-11), which is
 * not vendored in the reference; its call site is
 * production/dpa4c-runtime/components/deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:1497-1507
 * (run_model) reached from lammps-deepmd-plugin/src/pair_deepmd.cpp:370.
 * Each function below states the convention it fixes.
 */
#ifndef DPAMD_ORACLE_SE_E2_A_H
#define DPAMD_ORACLE_SE_E2_A_H
#include <stdint.h>

#define ORC_MAX_TYPES 8

typedef struct {
  int ntypes;
  int nnei;
  int sel[ORC_MAX_TYPES];
  int sec[ORC_MAX_TYPES + 1];
  double rcut, rcut_smth;
  int emb[3];   /* embedding widths L1, L2, L3 (M1 = L3) */
  int axis;     /* M2 */
  int fit[3];   /* fitting hidden widths */
  const double* davg;        /* [ntypes][ntypes][4]: per centre type, per neighbour section */
  const double* dstd;        /* [ntypes][ntypes][4] */
  const double* emb_params;  /* ntypes*ntypes blocks, see orc_emb_block_size */
  const double* fit_params;  /* ntypes blocks, see orc_fit_block_size */
  const double* bias_atom_e; /* [ntypes] */
} orc_model;

long orc_emb_block_size(const orc_model* m);
long orc_fit_block_size(const orc_model* m);

/* Ghost images of a periodic, LAMMPS-shaped (lower-triangular) box. */
int orc_ghost_count(int nloc, const double* coord, const double* box, double rcut);
int orc_build_ghosts(int nloc, const double* coord, const int* atype, const double* box,
                     double rcut, int nall_cap, double* ext_coord, int* ext_type, int* mapping);

/* Candidate lists (all j != i with r^2 <= rc^2), CSR by centre, sorted by j. */
long orc_candidates_brute(int nloc, int nall, const double* ext_coord, const int* ext_type,
                          double rc, long cap, long* offsets, int* cand);
long orc_candidates_cell(int nloc, int nall, const double* ext_coord, const int* ext_type,
                         const double* box, double rc, long cap, long* offsets, int* cand);

void orc_format_nlist(const orc_model* m, int nloc, const double* ext_coord, const int* ext_type,
                      const long* offsets, const int* cand, int* nlist);

void orc_env_mat(const orc_model* m, int nloc, const double* ext_coord, const int* ext_type,
                 const int* nlist, double* env, double* env_deriv, double* rij);

double orc_switch(double r, double rs, double rc, double* dsw);

void orc_embed(const orc_model* m, int ti, int tj, double s, double* g);

int orc_eval(const orc_model* m, int nloc, int nall, const double* ext_coord, const int* ext_type,
             const int* nlist, int nthreads, double* atom_energy, double* descrpt, double* dE_dD,
             double* net_deriv, double* edge_grad, double* force, double* virial, double* atom_virial);

void orc_prod_force(int nloc, int nall, int nnei, const double* ext_coord, const int* nlist,
                    const double* edge_grad, double* force, double* virial, double* atom_virial);

void orc_fold(int nloc, int nall, const int* mapping, const double* force_ext,
              const double* atom_virial_ext, double* force, double* atom_virial);

#endif
