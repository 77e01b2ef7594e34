// Kernel-side argument structs and host launchers of every pipeline stage.
#pragma once

#include <algorithm>
#include <mutex>

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
  int sel_strict;  // a section holding more than sel[t] atoms raises kStatusSelOverflow
  int unsorted;    // place candidates in candidate order instead of (type, r2, j) order
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
  double inv_sw;                 // 1 / (rcut - rcut_smth)
  // Precision-dependent arrays (double in fp64 mode, float in mixed mode):
  // emb, Tsec and dT; everything else is fp64 in both modes.
  const void* emb;     // [npair][stride] padded nets
  const double* envp;  // [npair][8] davg[4], dstd[4]
  const double* ext;   // [nall][3]
  const int* nlist;    // [nloc][nnei]
  const int* nreal;    // [nloc][ntypes]
  const int* items;    // centres grouped by type
  void* Tsec;          // forward out [nloc][ntypes][4][L3]
  const void* dT;      // backward in [nloc][4][L3]
  // Backward outputs. Each slot's edge gradient goes to its centre's
  // section sums cpsec [nloc][ntypes][12] (force 3, frame virial 9, fp64)
  // and, in fixed point (fixed.h), to its neighbour's extended-atom slot j:
  // facc [nall][3] and, when non-null, vacc [nall][9] (launch_fold_fixed
  // then moves ghost sums onto their owners). The forward clears both sums
  // at its end for the backward: zero_n atoms, or *zero_count when
  // zero_count is non-null.
  // edge_grad [nloc][nnei][3] is written only when non-null (kept for
  // inspection).
  double* edge_grad;
  unsigned long long* facc;
  unsigned long long* vacc;
  double* cpsec;
  long zero_n;
  const int* zero_count;
  // status word, and the largest |component| of an edge gradient the fixed
  // point accepts (raising kStatusFixedRange above it or on NaN)
  int* status;
  double fix_gmax;
  // Saved activations (fp64 kernels; the mixed backward recomputes them):
  // per (centre, tile of 16 slots) a block of 16*(L2P + L3P) doubles holding
  // tanh of layers 2 and 3 in the backward's register order; tiles of
  // section tj start at tile_off[tj], tiles_per_atom in total per centre.
  void* act;
  int tile_off[kMaxTypes + 1];
  int tiles_per_atom;
  // With a single neighbour type the forward writes T itself, (Tsec + npad
  // tpad) / nnei, into the column-major bucket layout Tt (element (pos, a, m)
  // at Tt[a * ldt + 4 pos + m]) instead of Tsec; null otherwise.
  void* Tt;
  long ldt;
  const double* tpad;  // [npair][4][L3]
  // items per wave: block b of a pair serves items (b ipw + k) WAVES + w,
  // k < ipw, so its weights are staged in LDS once for WAVES * ipw items
  int ipw;
};

struct DescArgs {
  int ntypes, nloc, L3, axis, nnei;
  int sel[kMaxTypes];
  double inv_nnei;
  const int* items;
  const int* ext_type;
  const int* nreal;
  const void* Tsec;    // element type of the mode (double / float)
  const double* tpad;  // [npair][4][L3]: Rpad[m] * Gpad[f], fp64 in both modes
  void* Tt;            // [L3][nloc][4] bucket order (T column-major)
  void* D;             // [nloc][L3*axis] bucket order, or null (not formed)
  int from_tt;         // T is already in Tt (written by the forward): only form D
};

// Neighbour stage
// also clears clear[0 .. nclear) and, when nall is given, sets *nall = nloc
void launch_wrap(hipStream_t, int nloc, const double* coord, const int* atype, const BoxParams&,
                 double* ext, int* ext_type, int* mapping, double* sfrac, int nclear, int* clear,
                 int* nall);
// Ghost images in (shift, atom) order: per shift, the number of images of each
// tile of atoms that land in the extended region (count[s * ghost_tiles(nloc)
// + tile]); then, from the exclusive scan of those counts, the images
// themselves (coordinates, types and mapping after the nloc local atoms).
int ghost_tiles(int nloc);
void launch_ghost_count(hipStream_t, int nloc, const BoxParams&, const double* sfrac, int* count);
// (also *nall = nloc + the number of ghosts)
void launch_ghost_place(hipStream_t, int nloc, const BoxParams&, const double* sfrac,
                        const int* count, const int* first, double* ext, int* ext_type,
                        int* mapping, int* nall);
// Cell kernels over cap atoms, or over *d_count of them when d_count is given
// (a count produced on the device, at most cap).
// (cell_rank: an atom's rank within its cell, from the count)
void launch_cell_assign(hipStream_t, int cap, const int* d_count, const BoxParams&,
                        const double* ext, int* cell_of, int* cell_rank, int* cell_count);
void launch_cell_scatter(hipStream_t, int cap, const int* d_count, const int* cell_of,
                         const int* cell_rank, const int* cell_start, const double* ext,
                         const int* ext_type, CellAtom* sorted);
// atoms of each cell in ascending index order (reproducible candidate order)
void launch_cell_order(hipStream_t, int ncell, const int* cell_start, CellAtom* sorted);
// p[0 .. n) = v (a kernel rather than a memset node, so it can be captured)
void launch_fill_int(hipStream_t, long n, int v, int* p);
// (sorted_cap: the capacity of `sorted` in records)
void launch_nlist_cells(hipStream_t, int nloc, const BoxParams&, const NlParams&, const double* ext,
                        const int* ext_type, const int* cell_of, const int* cell_start,
                        const CellAtom* sorted, long sorted_cap, int* nlist, int* nreal,
                        int* status);
void launch_nlist_csr(hipStream_t, int nloc, const NlParams&, const double* ext, const int* ext_type,
                      const long* cand_off, const int* cand, int* nlist, int* nreal, int* status);

// Edge-list front end (edges.hip): extended atoms nloc + e at the bond
// vectors, owners = source nodes, and the per-centre candidate counts
// (count must start at zero) and ranks; then the candidate CSR by centre.
template <class T>
void launch_edges_ext(hipStream_t, int nloc, int nedge, int nnode, const int* edge_index,
                      const T* edge_vec, const int* atype, double* ext, int* ext_type,
                      int* mapping, int* count, int* rank, int* status);
void launch_edges_fill(hipStream_t, int nloc, int nedge, int nnode, const int* edge_index,
                       const int* off, const int* rank, long* cand_off, int* cand);

// Static workspace of the no-allocation entry point (noalloc.hip): its size,
// and its address on `device` (which must be current), looked up once per
// device with hipGetSymbolAddress.
size_t noalloc_scratch_bytes();
void* noalloc_scratch_init(int device);
// The lock dp_compute_device_noalloc holds for a whole call on `device`.
std::mutex& noalloc_device_mutex(int device);

// Device-wide exclusive int prefix sums (scan.hip): scan_temp_bytes(n) of
// temporary device memory
size_t scan_temp_bytes(int n);
void exclusive_scan_int(hipStream_t, const int* in, int* out, int n, void* temp, size_t temp_bytes);

// Embedding stage. f32 selects the mixed-precision kernels (fp32 nets and
// contraction; env rows and edge gradients stay fp64), whose padded-net
// layout is make_emb_layout(L1, L2, L3, true).
bool emb_supported(int L1, int L2, int L3);
void launch_embed_fwd(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks, bool f32);
void launch_embed_bwd(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks, bool f32);
int embed_waves_fwd(const EmbLayout&, bool f32);
int embed_waves_bwd(const EmbLayout&, bool f32);
void launch_descriptor(hipStream_t, const DescArgs&, bool f32);
// fp32 embedding kernels (embed_f32.hip), reached through the two above
void launch_embed_fwd32(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks);
void launch_embed_bwd32(hipStream_t, const EmbLayout&, const EmbArgs&, int nblocks);
int embed_waves_fwd32(const EmbLayout&);
int embed_waves_bwd32(const EmbLayout&);

// Fitting stage, element type T = double (fp64 mode) or float (mixed mode);
// the energy head accumulates in fp64 in both.
template <class T>
struct FitLayer {
  const T* W;    // [in][out]
  const T* b;    // [out]
  const T* idt;  // [out] or null
  int in, out;
  // mixed precision: W (forward) and W^T (backward) pre-split into bf16
  // fragments for the fp32 GEMM on the bf16 matrix cores; null otherwise
  const void* Wf;
  const void* WfT;
};
template <class T>
struct FitNet {
  FitLayer<T> L[3];
  const T* Wo;   // [F2]
  double bo;
  double bias;   // bias_atom_e of the type
};
template <class T>
struct FitBufs {
  T *H0, *T1, *H1, *dZa, *dZb, *dH;  // [rows][F] each
  double* epart;  // [rows][F2 / column tile] partial energies of the head
  // first layer split over K into `split` slices (fit_splits) summed through
  // ws [split][rows][F0] when split > 1
  int split;
  T* ws;
};
// K slices fit_splits(rows, F0, Dn, compute units) for the first fitting layer
int fit_splits(int rows, int N, int K, int ncu);
// The first layer reads its input either from D ([rows][L3*axis]) or, when
// Tt is given (axis 16), forms D = T^T T[:, :16] on the fly from the
// column-major copy of T (element (row, a, m) at Tt[a * ldt + 4 row + m]) and
// D may be null.
// Without the fused kernel (fitting shapes other than F0 = 240, axis 16) the
// input gradient dD = dZ0 W0^T is a plain product of this library's GEMM.
// fp64: the first layer's input gradient fused with the descriptor backward
// (launch_dDdT); when given, launch_fitting computes dE/dT of its rows
// instead of dE/dD.
struct FitDdt {
  // first-layer weights: fp64 W0^T [F0][16 L3]; mixed precision the
  // tile-major bf16 pieces of W0^T (pack_gemm_bf16)
  const void* W0T;
  const int* items;   // bucket position -> atom
  int pos0;           // bucket position of the type's first row
  void* dT;           // [atoms][4][L3] (the net's precision)
  void* dD;           // [rows][16 L3] when kept for inspection, else null
  int ncu;
  // column-group splits (ddt_splits) and their workspace, (nsplit + 1) *
  // rows * 64 doubles (unused when nsplit == 1)
  int nsplit;
  double* ws;
};
int ddt_splits(int rows, int L3, int ncu);
bool ddt_supported(int F0, int L3, int axis);
void launch_dDdT(hipStream_t, int rows, int K, int L3, const double* dZ, const double* W0T,
                 const double* Tt, long ldt, int pos0, const int* items, double* dT, double* dD,
                 int ncu, int nsplit, double* ws);
void launch_dDdT3(hipStream_t, int rows, int K, int L3, const float* dZ, const void* W0f,
                  const float* Tt, long ldt, int pos0, const int* items, float* dT, float* dD,
                  int ncu, int nsplit, double* ws);
template <class T>
void launch_fitting(hipStream_t, const FitNet<T>&, int rows, const T* D, const T* Tt, long ldt,
                    int L3, const FitBufs<T>&, T* dD, double* e_bucket,
                    const FitDdt* ddt = nullptr);
// Tt column-major in bucket order (element (pos, a, m) at Tt[a * 4 nloc +
// 4 pos + m]), dT in atom order (items maps bucket position to atom).
template <class T>
void launch_dT(hipStream_t, int nloc, int L3, int axis, const int* items, const T* Tt, const T* dD,
               T* dT);

// Force / virial stage
// (rank: each edge's rank among the edges into its target, from the count)
void launch_rev_count(hipStream_t, long nedge, int nnei, const int* nlist, const int* mapping,
                      int* count, int* rank);
void launch_rev_fill(hipStream_t, long nedge, int nnei, const int* nlist, const int* mapping,
                     const int* off, const int* rank, int* rev);
// Fixed-point sums src of extended atoms j in [j0, n) added onto their
// owners mapping[j] in dst (integer atomics: order-independent); dst may be
// src when every owner lies below j0. n = *d_count when d_count is given (a
// count on the device, at most cap), else cap; src_v / dst_v may be null.
void launch_fold_fixed(hipStream_t, int j0, int cap, const int* d_count, const int* mapping,
                       const unsigned long long* src_f, const unsigned long long* src_v,
                       unsigned long long* dst_f, unsigned long long* dst_v);
// p[0 .. per * n) = 0 for 64-bit words, n = *d_count (at most cap) or cap
void launch_zero_u64(hipStream_t, long cap, const int* d_count, int per, unsigned long long* p);
// se_e2_a: forces, atom virials, energy and frame virial from the
// embedding backward's section sums cpsec [nloc][nsec][12] and the
// fixed-point target sums facc [ntarget][3], vacc [ntarget][9] (or null);
// type [nloc]: centres of a negative type have no sections. Per block of 256
// indices the bucket energies e_bucket [nbucket] and the centres' frame
// virials are summed into partials [finalize_ev_blocks(...)][10], then added
// in block order into out10 = [energy, virial[9]] (also written to energy /
// virial when given).
int finalize_ev_blocks(int ntarget, int nloc, int nbucket);
void launch_finalize_ev(hipStream_t, int ntarget, int nloc, int nbucket, int nsec, const int* type,
                        const double* cpsec, const unsigned long long* facc,
                        const unsigned long long* vacc, const double* e_bucket, double* force,
                        double* atom_virial, double* partials, double* out10, double* energy,
                        double* virial);
// cpart [nloc][12]: each centre's own-row force (3) and frame virial (9),
// written by the gather and summed by the reduction.
void launch_force_gather(hipStream_t, int ntarget, int nloc, int nnei, const int* rev_off,
                         const int* rev, const int* nlist, const double* ext,
                         const double* edge_grad, double* cpart, double* force,
                         double* atom_virial, int* status);
// out10 = [energy, virial[9]]; also written to energy / virial when given
void launch_reduce_ev(hipStream_t, int nbucket, int nloc, const double* atom_energy_bucket,
                      const double* cpart, double* partials, double* out10, double* energy,
                      double* virial);
void launch_scatter_energy(hipStream_t, int nloc, const int* items, const double* e_bucket,
                           double* atom_energy);

// DPA4C-Nano (dpa4c.hip). Per node the moments / cotangents are 44 floats:
// scalar [8], vector [3][4], tensor [5][4], the two envelope masses, 2 pad.
constexpr int kC4Mom = 44;
constexpr int kC4Out = 70;   // descriptor width
constexpr int kC4W0Ld = 72;  // row stride of the transposed first fitting layer
struct C4Params {
  const float* table;  // [n_int][6][8]: coefficient k of channel c at [i][k][c]
  const float* film;   // [nt*nt][8][2] PairFiLM (scale, shift)
  const float* ro;     // readout: Ma[4][4], Mt[4][4], Pv[4][4], Pt[4][2]
  const float* temb;   // [nt][8] type embedding
  const float* mean;   // [70]
  const float* istd;   // [70]
  const float* w0t;    // [H][kC4W0Ld] first fitting layer, transposed
  const float* b0;     // [H]
  const float* wh;     // [H] head
  const double* bias;  // [nt] bias_atom_e
  float bh;            // head bias
  int nt, n_int, H, act, resnet;
  float rcut, inv_rcut, eps2, floor, stride, inv_stride;
  int ncu;  // compute units: sizes the persistent edge-pass grids
};
// edges of a node from the sel-sorted list (standalone and LAMMPS paths)
struct C4Nlist {
  const int* nlist;  // [nloc][nnei]
  const int* nreal;  // [nloc][nt]
  const double* ext;
  const int* ext_type;
  int nnei;
  int sec[kMaxTypes + 1];
};
// edges of a node from a destination CSR of fp32 vectors (canonical graph)
struct C4Graph {
  const long* row_ptr;     // [nall + 1]
  const unsigned* source;  // [edges]
  const float* edge_vec;   // [edges][3] = x_src - x_dst
  const long* atype;       // [nall]
  long nall;
  long storage;            // edge slots; positions at or beyond are rejected
  int* status;
};
void launch_c4_moments(hipStream_t, const C4Params&, const C4Nlist&, int nnodes, float* mom,
                       int* status);
void launch_c4_moments(hipStream_t, const C4Params&, const C4Graph&, int nnodes, float* mom,
                       int* status);
void launch_c4_node(hipStream_t, const C4Params&, int nnodes, const int* type, const float* mom,
                    double* energy, float* cot);
void launch_c4_node(hipStream_t, const C4Params&, int nnodes, const long* type, const float* mom,
                    double* energy, float* cot);
// edge gradients dE/dd: [nloc][nnei][3] at the list's slots, or [edges][3]
void launch_c4_edge_grad(hipStream_t, const C4Params&, const C4Nlist&, int nnodes,
                         const float* cot, double* eg);
void launch_c4_edge_grad(hipStream_t, const C4Params&, const C4Graph&, int nnodes,
                         const float* cot, double* eg);
// standalone path: forces, atom virials (folded onto owners) and the
// centre-side partials cpart [nloc][12] from both directions of every edge
void launch_c4_edge_force(hipStream_t, const C4Params&, const C4Nlist&, int nnodes,
                          const int* mapping, const float* cot, double* force,
                          double* atom_virial, double* cpart);
void launch_c4_zero_tail(hipStream_t, const long* drow, int nloc, long storage, double* eg);
void launch_c4_graph_force(hipStream_t, int nall, const long* drow, const long* srow,
                           const unsigned* sorder, const float* edge_vec, const double* eg,
                           long storage, double* force, double* atom_virial, int* status);

}  // namespace dpamd
