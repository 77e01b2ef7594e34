// Kernel-side argument structs and host launchers of every pipeline stage.
#pragma once

#include "common.h"
#include "emb_shape.h"

namespace dpamd {

constexpr int kMaxCand = 512;  // candidates within rcut per centre held in LDS
constexpr int kMaxRev = 1024;  // edges pointing at one atom held in LDS
constexpr int kMaxPairs = kMaxTypes * kMaxTypes;

// Periodic cell (LAMMPS-shaped h) plus the cell grid over the extended region.
struct BoxParams {
  double h[9];
  double rcf[3];      // rcut in fractional units of each cell direction
  double hi[3];       // 1 + rcf
  int nrep[3];        // image shifts -nrep..nrep per direction
  int nshift;         // number of non-zero shifts
  int periodic;
  double origin[3];   // subtracted before the fractional transform (open systems)
  double cell_lo[3];  // fractional origin of the cell grid
  double cw[3];       // fractional cell width (>= rcut in perpendicular distance)
  int ncell[3];
};

struct NlParams {
  int ntypes, nnei;
  int sel[kMaxTypes];
  int sec[kMaxTypes + 1];
  double rc2;
};

struct CellAtom {
  double x, y, z;
  int idx, type;
};

// Embedding kernels (forward contraction and backward) share this bundle.
struct EmbArgs {
  int ntypes, nnei, npair;
  int sel[kMaxTypes];
  int sec[kMaxTypes + 1];
  int type_off[kMaxTypes + 1];   // bucket offsets of centres of each type
  int block_off[kMaxPairs + 1];  // first block of each (ti, tj) pair
  int stride;                    // doubles per padded net
  double rcut, rcut_smth, inv_nnei;
  const double* emb;   // [npair][stride] padded nets
  const double* envp;  // [npair][8] davg[4], dstd[4]
  const double* ext;   // [nall][3]
  const int* nlist;    // [nloc][nnei]
  const int* nreal;    // [nloc][ntypes]
  const int* items;    // centres grouped by type
  double* Tsec;        // forward out [nloc][ntypes][4][L3]
  const double* dT;    // backward in [nloc][4][L3]
  double* edge_grad;   // backward out [nloc][nnei][3]
  double* cpart;       // [nloc][ntypes][12]: centre force 3 + virial 9 (section 0 used)
  // Saved activations: per (centre, tile of 16 slots) a block of
  // 16*(L2P + L3P) doubles holding tanh of layers 2 and 3 in the backward's
  // register order; tiles of section tj start at tile_off[tj], tiles_per_atom
  // in total per centre.
  double* act;
  int tile_off[kMaxTypes + 1];
  int tiles_per_atom;
};

struct DescArgs {
  int ntypes, nloc, L3, axis, nnei;
  int sel[kMaxTypes];
  double inv_nnei;
  const int* items;
  const int* ext_type;
  const int* nreal;
  const double* Tsec;
  const double* tpad;  // [npair][4][L3]: Rpad[m] * Gpad[f]
  double* T;           // [nloc][4][L3] atom order
  double* D;           // [nloc][L3*axis] bucket order
};

// Neighbour stage
void launch_wrap(hipStream_t, int nloc, const double* coord, const int* atype, const BoxParams&,
                 double* ext, int* ext_type, int* mapping, double* sfrac);
void launch_ghost_flags(hipStream_t, int nloc, const BoxParams&, const double* sfrac, int* flags);
void launch_ghost_fill(hipStream_t, int nloc, const BoxParams&, const int* flags, const int* pos,
                       double* ext, int* ext_type, int* mapping);
void launch_cell_assign(hipStream_t, int nall, const BoxParams&, const double* ext, int* cell_of,
                        int* cell_count);
void launch_cell_scatter(hipStream_t, int nall, const int* cell_of, const int* cell_start,
                         int* cursor, const double* ext, const int* ext_type, CellAtom* sorted);
void launch_nlist_cells(hipStream_t, int nloc, const BoxParams&, const NlParams&, const double* ext,
                        const int* ext_type, const int* cell_of, const int* cell_start,
                        const CellAtom* sorted, int* nlist, int* nreal, int* status);
void launch_nlist_csr(hipStream_t, int nloc, const NlParams&, const double* ext, const int* ext_type,
                      const long* cand_off, const int* cand, int* nlist, int* nreal, int* status);

// Scans (hipCUB)
size_t scan_temp_bytes(int n);
void exclusive_scan_int(hipStream_t, const int* in, int* out, int n, void* temp, size_t temp_bytes);

// Embedding stage
bool emb_supported(int L1, int L2, int L3);
void launch_embed_fwd(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks);
void launch_embed_bwd(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks);
int embed_waves_fwd(const EmbLayout&);
int embed_waves_bwd(const EmbLayout&);
void launch_descriptor(hipStream_t, const DescArgs&);

// Fitting stage
struct FitLayer {
  const double* W;    // [in][out]
  const double* b;    // [out]
  const double* idt;  // [out] or null
  int in, out;
};
struct FitNet {
  FitLayer L[3];
  const double* Wo;  // [F2]
  double bo;
  double bias;       // bias_atom_e of the type
};
struct FitBufs {
  double *H0, *T1, *H1, *T2, *H2, *dZa, *dZb, *dH;  // [rows][F] each
};
void launch_fitting(hipStream_t, const FitNet&, int rows, const double* D, const FitBufs&,
                    double* dD, double* e_bucket);
void launch_dT(hipStream_t, int nloc, int L3, int axis, const int* items, const double* T,
               const double* dD, double* dT);

// Force / virial stage
void launch_rev_count(hipStream_t, long nedge, int nnei, const int* nlist, const int* mapping,
                      int* count);
void launch_rev_fill(hipStream_t, long nedge, int nnei, const int* nlist, const int* mapping,
                     const int* off, int* cursor, int* rev);
void launch_force_gather(hipStream_t, int ntarget, int nloc, int ntypes, int nnei,
                         const int* rev_off, const int* rev, const int* nlist, const double* ext,
                         const double* edge_grad, const double* cpart, double* force,
                         double* atom_virial, int* status);
void launch_center_sum(hipStream_t, int nloc, int ntypes, int nnei, const int* nlist,
                       const double* ext, const double* edge_grad, double* cpart);
void launch_reduce_ev(hipStream_t, int nbucket, int nloc, int ntypes,
                      const double* atom_energy_bucket, const double* cpart, double* partials,
                      double* out10);
void launch_scatter_energy(hipStream_t, int nloc, const int* items, const double* e_bucket,
                           double* atom_energy);

}  // namespace dpamd
