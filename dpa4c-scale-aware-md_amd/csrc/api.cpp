// C ABI of libdpamd.so and the per-step pipeline that drives the kernels.
//
// One evaluation (standalone path):
//   wrap + ghost images (count, scan, fill)          neighbor.hip
//   cell binning (count, scan, scatter)              neighbor.hip
//   sel-sorted neighbour list                        neighbor.hip
//   env mat + embedding + contraction -> Tsec        embed.hip   (FP64 MFMA)
//   descriptor T, D                                  embed.hip
//   fitting forward + input gradient per type        fitting.hip (FP64 MFMA)
//   dE/dD -> dE/dT                                   fitting.hip
//   embedding backward -> edge gradients             embed.hip   (FP64 MFMA)
//   reverse list + force / atom-virial gather        force.hip
//   energy / virial reduction                        force.hip
// The LAMMPS path replaces the first three stages with sel formatting of the
// caller's candidate list and keeps ghost forces in ghost slots. On the
// standalone device path no stage waits for the host: the ghost count stays
// on the device, and dp_compute_device_async only queues the evaluation
// (optionally as a replayed HIP graph), leaving capacity errors for dp_sync.
//
// This file is compiled with -ffp-contract=off: the box geometry (cutoff in
// fractional units) must match the oracle's bit for bit because it decides
// which ghost images exist.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/dp_amd.h"
#include "fixed.h"
#include "kernels.h"
#include "model.h"

using namespace dpamd;

namespace {

struct Buf {
  void* p = nullptr;
  size_t cap = 0;
};

enum Stage {
  kStGeom = 0,
  kStNlist,
  kStEmbFwd,
  kStDescr,
  kStFit,
  kStDT,
  kStEmbBwd,
  kStForce,
  kStReduce,
  kNumStages
};
const char* kStageNames[kNumStages] = {"ghost+cells", "nlist",  "embed_fwd",
                                       "descriptor",  "fitting", "dE_dT",
                                       "embed_bwd",   "force",  "reduce"};

}  // namespace

struct dp_model {
  int device = 0;
  int ncu = 256;  // compute units of the device
  int precision = DP_PREC_FP64;
  ModelHost host;
  // model kind: se_e2_a (DPAMDSEA files) or DPA4C-Nano (DPAMDC4N files)
  enum Kind { kSeA = 0, kDpa4c = 1 };
  int kind = kSeA;
  C4Host c4;
  C4Params c4p{};
  void* d_c4 = nullptr;  // every DPA4C parameter array, packed
  EmbLayout el{};
  std::string err;
  // device parameters; the nets (d_emb, d_fit) are double in fp64 mode and
  // float in mixed mode, env statistics and the padded-slot constant are fp64
  void* d_emb = nullptr;
  double* d_envp = nullptr;
  double* d_tpad = nullptr;
  void* d_fit = nullptr;
  // fp64: the first fitting layer's weights of every type transposed,
  // [nt][F0][L3 axis] (the fused dE/dD -> dE/dT kernel's operand), or null
  double* d_w0t = nullptr;
  // mixed precision: per type and fitting layer, byte offsets into d_fitf of
  // the pre-split W (forward) and W^T (backward) fragments, -1 if absent
  void* d_fitf = nullptr;
  long fitf_off[kMaxTypes][3][2];
  FitOffsets fo{};
  // With several centre types the per-type fitting chains run concurrently,
  // each on a stream of its own (default priority), forked from and joined
  // back into the evaluation stream.
  hipStream_t fit_st[kMaxTypes] = {};
  hipEvent_t fork_ev = nullptr;
  hipEvent_t join_ev[kMaxTypes] = {};
  // workspace
  std::vector<Buf*> bufs;
  Buf coord_in, atype_in, sfrac, flags, gpos, ext, ext_type, mapping, cell_of, cell_count,
      cell_start, cell_rank, sorted, nlist, nreal, cand_off, cand, items, Tsec, Tt, D, dD, dT,
      fitb, e_bucket, edge_grad, cpart, rev_count, rev_off, rev_rank, rev, force_ws, av_ws,
      ae_ws, partials, out10, status, scan_tmp, act, nall_d, split_ws, c4_mom, c4_cot, facc, vacc,
      cpsec, ftgt, vtgt, ddt_ws;
  size_t bytes_now = 0, bytes_peak = 0;
  // dp_compute_device_noalloc: buffers are carved from the device's static
  // scratch (noalloc.hip) instead of allocated; no stream forks, no vendor
  // library calls
  bool arena_on = false;
  char* arena_base = nullptr;
  size_t arena_cap = 0, arena_used = 0;
  // type buckets
  std::vector<int> atype_cache;
  std::vector<int> items_h;
  int type_off[kMaxTypes + 1] = {0};
  int nbucket = 0;
  bool buckets_valid = false;
  // LAMMPS candidate cache: the caller's list uploaded at ago == 0, valid
  // for the same nloc and nall until a rebuild (the edge entry points reuse
  // the same buffers and invalidate it)
  bool cand_valid = false;
  int cand_nloc = -1, cand_nall = -1;
  // last evaluation sizes (debug copies); on the standalone path last_nall is
  // the capacity of the extended arrays and the count itself is in nall_d
  int last_nloc = 0, last_nall = 0;
  bool last_standalone = true;
  // asynchronous evaluations (dp_compute_device_async): the status word is
  // sticky across them and copied to pinned host memory after each one
  int* status_host = nullptr;
  hipStream_t async_stream = nullptr;
  bool async_pending = false;
  // Graph replay of queued evaluations (DPAMD_GRAPH=1): the step is captured
  // once per key (sizes, pointers, box, stream, buffer and bucket
  // generations) on a stream of its own and replayed while the key holds.
  bool graph_on = false, graph_broken = false;
  hipStream_t graph_st = nullptr;
  hipEvent_t graph_in = nullptr, graph_out = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  std::vector<unsigned char> graph_key;
  int graph_warm = 0;
  long graph_captures = 0, graph_replays = 0;
  unsigned long buf_gen = 0, bucket_gen = 0;  // bumped by any reallocation / rebucketing
  // dp_debug_keep: store the per-slot edge gradients (which the se_e2_a
  // backward otherwise scatters without writing) for dp_debug_copy;
  // eg_valid: the last evaluation left them in edge_grad
  bool keep_edge_grad = false;
  bool eg_valid = false;
  // dp_debug_fused_rows: smallest type (rows) for which the fp64 fitting uses
  // the fused dE/dD -> dE/dT kernel
  int fused_ddt_rows = 12288;
  bool dd_valid = false;  // dE/dD of the last evaluation is in dD
  // stage timers
  bool timing = false;
  // one event set per evaluation in a ring, so that evaluations queued by
  // dp_compute_device_async are timed too; stage_ms is the mean over the
  // evaluations harvested since the previous synchronisation point
  static constexpr int kRing = 32;
  hipEvent_t ev[kRing][kNumStages + 1] = {};
  int ev_cur = 0, ev_head = 0, ev_pending = 0;
  double st_sum[kNumStages] = {0};
  int st_count = 0;
  float stage_ms[kNumStages] = {0};

  dp_model() {
    bufs = {&coord_in, &atype_in, &sfrac,     &flags,    &gpos,       &ext,       &ext_type,
            &mapping,  &cell_of,  &cell_count, &cell_start, &cell_rank, &sorted,   &nlist,
            &nreal,    &cand_off, &cand,      &items,    &Tsec,       &Tt,        &D,
            &dD,       &dT,       &fitb,      &e_bucket, &edge_grad,  &cpart,     &rev_count,
            &rev_off,  &rev_rank, &rev,       &force_ws, &av_ws,      &ae_ws,     &partials,
            &out10,    &status,   &scan_tmp, &act,       &nall_d,    &split_ws,  &c4_mom,
            &c4_cot,   &facc,     &vacc,      &cpsec,      &ftgt,      &vtgt,      &ddt_ws};
  }
};

namespace {

struct ApiError;
[[noreturn]] void arena_full(dp_model* M, size_t bytes);

template <class T>
T* need(dp_model* M, Buf& b, size_t count) {
  const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
  if (M->arena_on) {
    // carve from the static scratch (256-byte aligned); a buffer asked for
    // again with a larger size gets a new region
    if (b.p && bytes <= b.cap) return static_cast<T*>(b.p);
    const size_t off = (M->arena_used + 255) & ~size_t(255);
    if (off + bytes > M->arena_cap) arena_full(M, off + bytes);
    b.p = M->arena_base + off;
    b.cap = bytes;
    M->arena_used = off + bytes;
    return static_cast<T*>(b.p);
  }
  if (bytes > b.cap) {
    if (b.p) {
      // queued asynchronous evaluations may still use the old buffer
      if (M->async_pending) DPAMD_HIP(hipStreamSynchronize(M->async_stream));
      DPAMD_HIP(hipFree(b.p));
      M->bytes_now -= b.cap;
    }
    const size_t nb = bytes + bytes / 8;
    b.p = nullptr;
    b.cap = 0;
    DPAMD_HIP(hipMalloc(&b.p, nb));
    b.cap = nb;
    ++M->buf_gen;
    M->bytes_now += nb;
    M->bytes_peak = std::max(M->bytes_peak, M->bytes_now);
  }
  return static_cast<T*>(b.p);
}

struct ApiError {
  int code;
  std::string msg;
};

void arena_full(dp_model* M, size_t bytes) {
  throw ApiError{DP_ERR_CAPACITY,
                 "the system needs more than the " + std::to_string(M->arena_cap >> 20) +
                     " MiB of static scratch of dp_compute_device_noalloc (at least " +
                     std::to_string((bytes + (1 << 20) - 1) >> 20) +
                     " MiB); use dp_compute_device"};
}

// LAMMPS-shaped periodic box; formulas identical to the oracle's box_geometry.
BoxParams make_box(const double* box, double rcut) {
  BoxParams bp{};
  for (int q = 0; q < 9; ++q) bp.h[q] = box[q];
  const double xx = box[0], xy = box[3], yy = box[4], xz = box[6], yz = box[7], zz = box[8];
  if (box[1] != 0.0 || box[2] != 0.0 || box[5] != 0.0)
    throw ApiError{DP_ERR_ARG, "box must be lower-triangular (LAMMPS h: box[1]=box[2]=box[5]=0)"};
  if (!(xx > 0.0 && yy > 0.0 && zz > 0.0))
    throw ApiError{DP_ERR_ARG, "box diagonal must be positive"};
  const double vol = xx * yy * zz;
  const double bc0 = yy * zz, bc1 = xy * zz, bc2 = xy * yz - yy * xz;
  const double ha = vol / std::sqrt(bc0 * bc0 + bc1 * bc1 + bc2 * bc2);
  const double hb = (yy * zz) / std::sqrt(zz * zz + yz * yz);
  const double hc = zz;
  bp.rcf[0] = rcut / ha;
  bp.rcf[1] = rcut / hb;
  bp.rcf[2] = rcut / hc;
  for (int d = 0; d < 3; ++d) {
    bp.nrep[d] = (int)std::ceil(bp.rcf[d]);
    bp.hi[d] = 1.0 + bp.rcf[d];
    bp.origin[d] = 0.0;
    bp.cell_lo[d] = -bp.rcf[d];
    const double extent = 1.0 + 2.0 * bp.rcf[d];
    int nc = (int)std::floor(extent / (bp.rcf[d] * (1.0 + 1e-6)));
    nc = std::max(1, std::min(nc, 256));
    bp.ncell[d] = nc;
    bp.cw[d] = extent / nc;
  }
  bp.nshift = (2 * bp.nrep[0] + 1) * (2 * bp.nrep[1] + 1) * (2 * bp.nrep[2] + 1) - 1;
  bp.periodic = 1;
  return bp;
}

// Open system: a synthetic orthorhombic frame only for cell binning.
BoxParams make_open_frame(int n, const double* coord, double rcut) {
  BoxParams bp{};
  double lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
  for (int d = 0; d < 3; ++d) {
    lo[d] = n ? coord[d] : 0.0;
    hi[d] = lo[d];
  }
  for (int k = 0; k < n; ++k)
    for (int d = 0; d < 3; ++d) {
      lo[d] = std::min(lo[d], coord[3 * k + d]);
      hi[d] = std::max(hi[d], coord[3 * k + d]);
    }
  for (int d = 0; d < 3; ++d) {
    const double L = (hi[d] - lo[d]) + 2.0;
    bp.h[4 * d] = L;
    bp.origin[d] = lo[d] - 1.0;
    bp.rcf[d] = rcut / L;
    bp.cell_lo[d] = 0.0;
    int nc = (int)std::floor(1.0 / (bp.rcf[d] * (1.0 + 1e-6)));
    nc = std::max(1, std::min(nc, 256));
    bp.ncell[d] = nc;
    bp.cw[d] = 1.0 / nc;
  }
  bp.nshift = 0;
  bp.periodic = 0;
  return bp;
}

void record(dp_model* M, hipStream_t st, int stage) {
  if (M->timing) DPAMD_HIP(hipEventRecord(M->ev[M->ev_cur][stage], st));
}

// Group centres by type (stable) when the types change.
void update_buckets(dp_model* M, int nloc, const int* atype_host, hipStream_t st) {
  const int nt = M->host.ntypes;
  if (M->buckets_valid && (int)M->atype_cache.size() == nloc &&
      std::equal(atype_host, atype_host + nloc, M->atype_cache.begin()))
    return;
  M->atype_cache.assign(atype_host, atype_host + nloc);
  M->items_h.clear();
  M->items_h.reserve(nloc);
  for (int t = 0; t < nt; ++t) {
    M->type_off[t] = (int)M->items_h.size();
    for (int k = 0; k < nloc; ++k)
      if (atype_host[k] == t) M->items_h.push_back(k);
  }
  M->type_off[nt] = (int)M->items_h.size();
  M->nbucket = M->type_off[nt];
  ++M->bucket_gen;
  int* d_items = need<int>(M, M->items, std::max(1, M->nbucket));
  if (M->nbucket)
    DPAMD_HIP(hipMemcpyAsync(d_items, M->items_h.data(), sizeof(int) * M->nbucket,
                             hipMemcpyHostToDevice, st));
  DPAMD_HIP(hipStreamSynchronize(st));
  M->buckets_valid = true;
}

struct Outputs {
  double* energy;       // device [1] or null
  double* force;        // device [ntarget][3]
  double* virial;       // device [9] or null
  double* atom_energy;  // device [ntarget] or null
  double* atom_virial;  // device [ntarget][9] or null
};

// Everything after the neighbour list; ext/ext_type/nlist/nreal/mapping ready.
// Arguments of the descriptor kernel for the current buckets: T (and D when
// non-null) in bucket order from Tsec.
DescArgs desc_args(dp_model* M, void* Tt, void* D) {
  const ModelHost& m = M->host;
  DescArgs da{};
  da.ntypes = m.ntypes;
  da.nloc = M->nbucket;
  da.L3 = m.emb[2];
  da.axis = m.axis;
  da.nnei = m.nnei;
  for (int t = 0; t < m.ntypes; ++t) da.sel[t] = m.sel[t];
  da.inv_nnei = 1.0 / (double)m.nnei;
  da.items = static_cast<const int*>(M->items.p);
  da.ext_type = static_cast<const int*>(M->ext_type.p);
  da.nreal = static_cast<const int*>(M->nreal.p);
  da.Tsec = M->Tsec.p;
  da.tpad = M->d_tpad;
  da.Tt = Tt;
  da.D = D;
  da.from_tt = m.ntypes == 1;  // the forward wrote T itself
  return da;
}

void gather_and_reduce(dp_model* M, hipStream_t st, int nloc, int ntarget, const int* d_mapping,
                       const double* e_vals, int ne, const int* items, const Outputs& out);
void reduce_outputs(dp_model* M, hipStream_t st, int nloc, int ntarget, const double* e_vals,
                    int ne, const int* items, const Outputs& out);
void atom_energy_out(dp_model* M, hipStream_t st, int ntarget, const double* e_vals, int ne,
                     const int* items, const Outputs& out);

// nall: extended atoms, or (d_nall non-null, standalone path) their
// capacity with the count itself on the device.
template <class E>
void run_model_t(dp_model* M, hipStream_t st, int nloc, int nall, const int* d_nall,
                 const int* d_mapping, int ntarget, const Outputs& out) {
  constexpr bool f32 = sizeof(E) == 4;
  const ModelHost& m = M->host;
  const int nt = m.ntypes, nnei = m.nnei, L3 = m.emb[2], axis = m.axis, Dn = L3 * axis;
  const int nb = M->nbucket;
  const double* ext = static_cast<const double*>(M->ext.p);
  const int* nlist = static_cast<const int*>(M->nlist.p);
  const int* nreal = static_cast<const int*>(M->nreal.p);
  const int* items = static_cast<const int*>(M->items.p);

  E* Tsec = need<E>(M, M->Tsec, (size_t)nloc * nt * 4 * L3);
  // T column-major in bucket order; with axis 16 the first fitting GEMM forms
  // D from it, otherwise D is stored
  E* Tt = need<E>(M, M->Tt, (size_t)std::max(nb, 1) * 4 * L3);
  const bool d_from_t = axis == 16;
  E* D = d_from_t ? nullptr : need<E>(M, M->D, (size_t)std::max(nb, 1) * Dn);
  // fp64 with the fused input-gradient kernel: dE/dD is not stored (only
  // when kept for inspection). In fp64 a type of few rows gives the fused
  // kernel too few blocks (it splits its column groups instead), and the
  // plain product dE/dD = dZ0 W0^T followed by the dE/dT pass is faster:
  // water-5k 1.09 -> 1.01 ms/step, water-12k 1.96 -> 1.90; equal at 24k and
  // slower from 98k (queued steps, one box). So fp64 takes the fused kernel
  // when every type has at least fused_ddt_rows rows.
  int min_rows = nb;
  for (int t = 0; t < nt; ++t) {
    const int rows = M->type_off[t + 1] - M->type_off[t];
    if (rows > 0) min_rows = std::min(min_rows, rows);
  }
  const bool fused_ddt =
      d_from_t && (f32 ? M->fitf_off[0][0][1] >= 0
                       : M->d_w0t != nullptr && min_rows >= M->fused_ddt_rows);
  E* dD = (!fused_ddt || M->keep_edge_grad) ? need<E>(M, M->dD, (size_t)std::max(nb, 1) * Dn)
                                            : nullptr;
  E* dT = need<E>(M, M->dT, (size_t)nloc * 4 * L3);
  const int Fmax = std::max(m.fit[0], std::max(m.fit[1], m.fit[2]));
  // six activation slabs [nb][Fmax] and the head's partial energies
  // [nb][F2 / 16] fp64 (no larger than one slab of E)
  E* fitb = need<E>(M, M->fitb, (size_t)7 * std::max(nb, 1) * Fmax);
  double* e_bucket = need<double>(M, M->e_bucket, (size_t)std::max(nb, 1));
  // the backward scatters each edge's forces itself (fixed point) and stores
  // g only when kept
  double* edge_grad = M->keep_edge_grad
                          ? need<double>(M, M->edge_grad, (size_t)std::max(nloc, 1) * nnei * 3)
                          : nullptr;
  const long nfix = std::max(nall, ntarget);
  auto* facc = need<unsigned long long>(M, M->facc, (size_t)std::max(nfix, 1L) * 3);
  auto* vacc = out.atom_virial
                   ? need<unsigned long long>(M, M->vacc, (size_t)std::max(nfix, 1L) * 9)
                   : nullptr;
  double* cpsec = need<double>(M, M->cpsec, (size_t)std::max(nloc, 1) * nt * 12);

  EmbArgs ea{};
  ea.ntypes = nt;
  ea.nnei = nnei;
  ea.npair = nt * nt;
  for (int t = 0; t < nt; ++t) ea.sel[t] = m.sel[t];
  for (int t = 0; t <= nt; ++t) {
    ea.sec[t] = m.sec[t];
    ea.type_off[t] = M->type_off[t];
  }
  ea.stride = M->el.stride;
  ea.rcut = m.rcut;
  ea.rcut_smth = m.rcut_smth;
  ea.inv_sw = 1.0 / (m.rcut - m.rcut_smth);
  ea.status = static_cast<int*>(M->status.p);
  ea.fix_gmax = fixed_gmax(m.rcut);
  ea.inv_nnei = 1.0 / (double)nnei;
  ea.emb = M->d_emb;
  ea.envp = M->d_envp;
  ea.ext = ext;
  ea.nlist = nlist;
  ea.nreal = nreal;
  ea.items = items;
  ea.Tsec = Tsec;
  ea.dT = dT;
  ea.edge_grad = edge_grad;
  ea.facc = facc;
  ea.vacc = vacc;
  ea.cpsec = cpsec;
  // the fixed-point sums are cleared by the forward (no kernel of their own;
  // stores, not a memset, so the step can be captured in a graph); on the
  // standalone path over the ghosts counted on the device
  ea.zero_n = nfix;
  ea.zero_count = d_nall;
  ea.Tt = nt == 1 ? static_cast<void*>(Tt) : nullptr;
  ea.ldt = 4L * nb;
  ea.tpad = M->d_tpad;
  {
    int acc = 0;
    for (int t = 0; t < nt; ++t) {
      ea.tile_off[t] = acc;
      acc += (m.sel[t] + 15) / 16;
    }
    ea.tile_off[nt] = acc;
    ea.tiles_per_atom = acc;
    // fp64: the forward saves the layer-2/3 activations for the backward;
    // mixed precision recomputes them there (no buffer)
    const size_t blk = 16 * (size_t)(M->el.L2P + M->el.L3P);
    ea.act = f32 ? nullptr : need<E>(M, M->act, (size_t)std::max(nloc, 1) * acc * blk);
  }
  // Blocks of WAVES * ipw items: each block stages its pair's net in LDS once
  // and its waves then walk ipw items each, which amortises the staging and
  // the start-up latency of a block. ipw aims at about 32 tiles of 16 slots
  // per wave, as long as the grid still gives every compute unit six blocks
  // or more: the blocks of different pairs differ in length, and with few
  // blocks per unit the last ones leave a tail where some units idle
  // (12,288-atom water, per-block timestamps: 12 % of the units' time idle
  // with three blocks per unit; six: embedding kernels -9 %).
  auto block_table = [&](int waves) {
    long items = 0;
    for (int p = 0; p < nt * nt; ++p) items += M->type_off[p / nt + 1] - M->type_off[p / nt];
    const long tiles = std::max(1, (ea.tiles_per_atom + nt - 1) / nt);  // per item
    const long by_tiles = (32 + tiles - 1) / tiles;
    const long by_grid = items / ((long)waves * 6 * M->ncu);
    ea.ipw = (int)std::clamp(std::min(by_tiles, by_grid), 1L, 16L);
    const int per = waves * ea.ipw;
    int acc = 0;
    for (int p = 0; p < nt * nt; ++p) {
      ea.block_off[p] = acc;
      const int ti = p / nt;
      const int cnt = M->type_off[ti + 1] - M->type_off[ti];
      acc += (cnt + per - 1) / per;
    }
    ea.block_off[nt * nt] = acc;
    return acc;
  };

  int nblk = block_table(embed_waves_fwd(M->el, f32));
  launch_embed_fwd(st, M->el, ea, nblk, f32);
  if (nblk <= 0) {
    // no forward grid to clear the fixed-point sums (no centres)
    launch_zero_u64(st, ea.zero_n, ea.zero_count, 3, facc);
    if (vacc) launch_zero_u64(st, ea.zero_n, ea.zero_count, 9, vacc);
  }
  record(M, st, kStEmbFwd + 1);

  if (nt > 1 || D) launch_descriptor(st, desc_args(M, Tt, D), f32);
  record(M, st, kStDescr + 1);

  int active = 0;
  size_t ws_need = 0, ws_off = 0, ddt_need = 0, ddt_off = 0;
  for (int t = 0; t < nt; ++t) {
    const int rows = M->type_off[t + 1] - M->type_off[t];
    active += rows > 0;
    const int sp = rows > 0 ? fit_splits(rows, m.fit[0], Dn, M->ncu) : 1;
    if (sp > 1) ws_need += (size_t)sp * rows * m.fit[0];
    const int ds = (fused_ddt && rows > 0) ? ddt_splits(rows, L3, M->ncu) : 1;
    if (ds > 1) ddt_need += (size_t)(ds + 1) * rows * 64;
  }
  // the fused input-gradient kernel's split partials, one region per type
  double* ddt_ws = ddt_need ? need<double>(M, M->ddt_ws, ddt_need) : nullptr;
  // split-K slices of the first layer, one region per type (the chains run
  // concurrently)
  E* split_ws = ws_need ? need<E>(M, M->split_ws, ws_need) : nullptr;
  const bool fork = active > 1 && !M->arena_on;
  // With the plain dE/dD product (few rows per type) the type with the most
  // rows stays on the evaluation stream, enqueued last, and only the others
  // wait for the fork event (water-12k 1.95 -> 1.91 ms/step); with the fused
  // kernel every type runs on a stream of its own (keeping one on the
  // evaluation stream measured 0.3-0.7 % slower on HEA-128k and water-393k).
  int tmain = -1;
  if (fork && !fused_ddt) {
    tmain = 0;
    for (int t = 1; t < nt; ++t)
      if (M->type_off[t + 1] - M->type_off[t] > M->type_off[tmain + 1] - M->type_off[tmain])
        tmain = t;
  }
  if (fork) {
    if (!M->fork_ev) DPAMD_HIP(hipEventCreateWithFlags(&M->fork_ev, hipEventDisableTiming));
    DPAMD_HIP(hipEventRecord(M->fork_ev, st));
  }
  for (int q = 0; q < nt; ++q) {
    // visiting order: every type but tmain, then tmain
    const int t = tmain < 0 ? q : (q < tmain ? q : (q + 1 < nt ? q + 1 : tmain));
    const int rows = M->type_off[t + 1] - M->type_off[t];
    if (rows <= 0) continue;
    const bool side = fork && t != tmain;
    hipStream_t fst = st;
    if (side) {
      if (!M->fit_st[t]) {
        DPAMD_HIP(hipStreamCreateWithFlags(&M->fit_st[t], hipStreamNonBlocking));
        DPAMD_HIP(hipEventCreateWithFlags(&M->join_ev[t], hipEventDisableTiming));
      }
      fst = M->fit_st[t];
      DPAMD_HIP(hipStreamWaitEvent(fst, M->fork_ev, 0));
    }
    const E* P = static_cast<const E*>(M->d_fit) + (size_t)t * m.fit_block;
    FitNet<E> net{};
    const int ins[3] = {Dn, m.fit[0], m.fit[1]};
    for (int k = 0; k < 3; ++k) {
      net.L[k].W = P + M->fo.W[k];
      net.L[k].b = P + M->fo.b[k];
      net.L[k].idt = M->fo.idt[k] >= 0 ? P + M->fo.idt[k] : nullptr;
      net.L[k].in = ins[k];
      net.L[k].out = m.fit[k];
      if (f32 && M->d_fitf) {
        const char* fb = static_cast<const char*>(M->d_fitf);
        net.L[k].Wf = M->fitf_off[t][k][0] >= 0 ? fb + M->fitf_off[t][k][0] : nullptr;
        net.L[k].WfT = M->fitf_off[t][k][1] >= 0 ? fb + M->fitf_off[t][k][1] : nullptr;
      }
    }
    net.Wo = P + M->fo.Wo;
    net.bo = m.fit_params[(size_t)t * m.fit_block + M->fo.bo];
    net.bias = m.bias[t];
    const size_t r0 = (size_t)M->type_off[t];
    const size_t slab = (size_t)std::max(nb, 1) * Fmax;
    FitBufs<E> fb{};
    fb.split = fit_splits(rows, m.fit[0], Dn, M->ncu);
    if (fb.split > 1) fb.ws = split_ws + ws_off;
    ws_off += (size_t)fb.split * rows * m.fit[0];
    E* base = fitb;
    E** slots[6] = {&fb.H0, &fb.T1, &fb.H1, &fb.dZa, &fb.dZb, &fb.dH};
    // slab q holds [rows][F] of every type back to back; F <= Fmax. Slab 6
    // holds the head's partial energies (at most F2 / 16 doubles per row).
    for (int q = 0; q < 6; ++q) *slots[q] = base + q * slab + r0 * (size_t)Fmax;
    fb.epart = reinterpret_cast<double*>(base + 6 * slab) + r0 * (size_t)(m.fit[2] / 16);
    FitDdt ddt{};
    if (fused_ddt) {
      if constexpr (f32)
        ddt.W0T = static_cast<const char*>(M->d_fitf) + M->fitf_off[t][0][1];
      else
        ddt.W0T = M->d_w0t + (size_t)t * m.fit[0] * Dn;
      ddt.items = items;
      ddt.pos0 = (int)r0;
      ddt.dT = dT;
      ddt.dD = dD ? dD + r0 * Dn : nullptr;
      ddt.ncu = M->ncu;
      ddt.nsplit = ddt_splits(rows, L3, M->ncu);
      ddt.ws = ddt.nsplit > 1 ? ddt_ws + ddt_off : nullptr;
      if (ddt.nsplit > 1) ddt_off += (size_t)(ddt.nsplit + 1) * rows * 64;
    }
    launch_fitting(fst, net, rows, d_from_t ? nullptr : D + r0 * Dn,
                   d_from_t ? Tt + r0 * 4 : nullptr, 4L * nb, L3, fb, dD ? dD + r0 * Dn : nullptr,
                   e_bucket + r0, fused_ddt ? &ddt : nullptr);
    if (side) DPAMD_HIP(hipEventRecord(M->join_ev[t], fst));
  }
  if (fork)
    for (int t = 0; t < nt; ++t)
      if (t != tmain && M->type_off[t + 1] > M->type_off[t])
        DPAMD_HIP(hipStreamWaitEvent(st, M->join_ev[t], 0));
  record(M, st, kStFit + 1);

  if (!fused_ddt) launch_dT(st, nb, L3, axis, items, Tt, dD, dT);
  M->dd_valid = dD != nullptr;
  record(M, st, kStDT + 1);

  // (the fixed-point sums were cleared by the forward)
  nblk = block_table(embed_waves_bwd(M->el, f32));
  launch_embed_bwd(st, M->el, ea, nblk, f32);
  M->eg_valid = edge_grad != nullptr;
  record(M, st, kStEmbBwd + 1);
  const int nsec = nt;
  const unsigned long long *fsum = facc, *vsum = vacc;
  if (d_mapping && ntarget == nloc) {
    // every owner is local: ghost sums folded in place
    launch_fold_fixed(st, nloc, nall, d_nall, d_mapping, facc, vacc, facc, vacc);
  } else if (d_mapping) {
    // owners beyond the locals (the edge graph's kept ghost nodes) share
    // indices with extended atoms: fold every atom into separate target sums
    auto* ft = need<unsigned long long>(M, M->ftgt, (size_t)std::max(ntarget, 1) * 3);
    auto* vt = vacc ? need<unsigned long long>(M, M->vtgt, (size_t)std::max(ntarget, 1) * 9) : nullptr;
    launch_zero_u64(st, ntarget, nullptr, 3, ft);
    if (vt) launch_zero_u64(st, ntarget, nullptr, 9, vt);
    launch_fold_fixed(st, 0, nall, d_nall, d_mapping, facc, vacc, ft, vt);
    fsum = ft;
    vsum = vt;
  }
  // forces and atom virials, then energy and frame virial (both stages of the
  // reduction under the force timer)
  double* partials =
      need<double>(M, M->partials, (size_t)finalize_ev_blocks(ntarget, nloc, nb) * 10);
  double* out10 = need<double>(M, M->out10, 10);
  launch_finalize_ev(st, ntarget, nloc, nb, nsec, static_cast<const int*>(M->ext_type.p), cpsec,
                     fsum, vsum, e_bucket, out.force, out.atom_virial, partials, out10, out.energy,
                     out.virial);
  record(M, st, kStForce + 1);
  atom_energy_out(M, st, ntarget, e_bucket, nb, items, out);
}

// Reverse list + force / atom-virial gather from stored edge gradients (the
// DPA4C edge-gradient paths: the LAMMPS list and the edge-graph entries),
// then the energy / virial reduction. Atom
// energies e_vals[0..ne) are in bucket order (items maps a position to its
// atom) or, with items null, in atom order.
void gather_and_reduce(dp_model* M, hipStream_t st, int nloc, int ntarget, const int* d_mapping,
                       const double* e_vals, int ne, const int* items, const Outputs& out) {
  const int nnei = M->host.nnei;
  const int* nlist = static_cast<const int*>(M->nlist.p);
  const double* ext = static_cast<const double*>(M->ext.p);
  const double* edge_grad = static_cast<const double*>(M->edge_grad.p);
  int* status = static_cast<int*>(M->status.p);
  double* cpart = need<double>(M, M->cpart, (size_t)std::max(nloc, 1) * 12);
  const long nedge = (long)nloc * nnei;
  int* rcount = need<int>(M, M->rev_count, (size_t)ntarget + 1);
  int* roff = need<int>(M, M->rev_off, (size_t)ntarget + 1);
  int* rrank = need<int>(M, M->rev_rank, (size_t)std::max<long>(nedge, 1));
  int* rev = need<int>(M, M->rev, (size_t)std::max<long>(nedge, 1));
  launch_fill_int(st, (long)ntarget + 1, 0, rcount);
  launch_rev_count(st, nedge, nnei, nlist, d_mapping, rcount, rrank);
  {
    const size_t tb = scan_temp_bytes(ntarget + 1);
    void* tmp = need<char>(M, M->scan_tmp, tb);
    exclusive_scan_int(st, rcount, roff, ntarget + 1, tmp, tb);
  }
  launch_rev_fill(st, nedge, nnei, nlist, d_mapping, roff, rrank, rev);
  launch_force_gather(st, ntarget, nloc, nnei, roff, rev, nlist, ext, edge_grad, cpart,
                      out.force, out.atom_virial, status);
  record(M, st, kStForce + 1);
  reduce_outputs(M, st, nloc, ntarget, e_vals, ne, items, out);
}

// Energy and frame virial from the atom energies and the centre partials
// cpart, copied into the caller's outputs.
void reduce_outputs(dp_model* M, hipStream_t st, int nloc, int ntarget, const double* e_vals,
                    int ne, const int* items, const Outputs& out) {
  const double* cpart = static_cast<const double*>(M->cpart.p);
  double* partials = need<double>(M, M->partials, 256 * 10);
  double* out10 = need<double>(M, M->out10, 10);
  launch_reduce_ev(st, ne, nloc, e_vals, cpart, partials, out10, out.energy, out.virial);
  atom_energy_out(M, st, ntarget, e_vals, ne, items, out);
}

// Atom energies (when asked for) from e_vals[0..ne), in bucket order (items
// maps a position to its atom) or, with items null, in atom order; the
// reduce stage timer.
void atom_energy_out(dp_model* M, hipStream_t st, int ntarget, const double* e_vals, int ne,
                     const int* items, const Outputs& out) {
  if (out.atom_energy) {
    launch_fill_int(st, 2L * ntarget, 0, reinterpret_cast<int*>(out.atom_energy));
    if (items) {
      launch_scatter_energy(st, ne, items, e_vals, out.atom_energy);
    } else if (ne > 0) {
      DPAMD_HIP(hipMemcpyAsync(out.atom_energy, e_vals, sizeof(double) * ne,
                               hipMemcpyDeviceToDevice, st));
    }
  }
  record(M, st, kStReduce + 1);
}

// DPA4C-Nano on the sel-sorted list: moments, node pass (readout, fitting,
// readout VJP), then on the standalone path one edge pass straight into
// forces and virials, on the LAMMPS path (ghost slots kept) edge gradients,
// the shared gather and the reduction. Stage timers: moments under embed_fwd,
// the node pass under fitting, edge gradients under embed_bwd, the fused
// edge/force pass under force.
void run_c4(dp_model* M, hipStream_t st, int nloc, const int* d_mapping, int ntarget,
            const Outputs& out, bool complete) {
  const ModelHost& m = M->host;
  C4Nlist src{};
  src.nlist = static_cast<const int*>(M->nlist.p);
  src.nreal = static_cast<const int*>(M->nreal.p);
  src.ext = static_cast<const double*>(M->ext.p);
  src.ext_type = static_cast<const int*>(M->ext_type.p);
  src.nnei = m.nnei;
  for (int t = 0; t <= m.ntypes; ++t) src.sec[t] = m.sec[t];
  int* status = static_cast<int*>(M->status.p);
  float* mom = need<float>(M, M->c4_mom, (size_t)std::max(nloc, 1) * kC4Mom);
  float* cot = need<float>(M, M->c4_cot, (size_t)std::max(nloc, 1) * kC4Mom);
  double* e = need<double>(M, M->e_bucket, (size_t)std::max(nloc, 1));
  launch_c4_moments(st, M->c4p, src, nloc, mom, status);
  record(M, st, kStEmbFwd + 1);
  record(M, st, kStDescr + 1);
  launch_c4_node(st, M->c4p, nloc, src.ext_type, mom, e, cot);
  record(M, st, kStFit + 1);
  record(M, st, kStDT + 1);
  if (complete) {
    // standalone: the list is complete and folded onto owners, so both
    // directions of each edge are evaluated by its centre (no reverse list)
    record(M, st, kStEmbBwd + 1);
    double* cpart = need<double>(M, M->cpart, (size_t)std::max(nloc, 1) * 12);
    launch_c4_edge_force(st, M->c4p, src, nloc, d_mapping, cot, out.force, out.atom_virial,
                         cpart);
    M->eg_valid = false;
    record(M, st, kStForce + 1);
    double* partials = need<double>(M, M->partials, 256 * 10);
    double* out10 = need<double>(M, M->out10, 10);
    launch_reduce_ev(st, nloc, nloc, e, cpart, partials, out10, out.energy, out.virial);
    if (out.atom_energy && nloc > 0)
      DPAMD_HIP(hipMemcpyAsync(out.atom_energy, e, sizeof(double) * nloc,
                               hipMemcpyDeviceToDevice, st));
    record(M, st, kStReduce + 1);
    (void)ntarget;
    return;
  }
  double* eg = need<double>(M, M->edge_grad, (size_t)std::max(nloc, 1) * m.nnei * 3);
  launch_c4_edge_grad(st, M->c4p, src, nloc, cot, eg);
  M->eg_valid = true;
  record(M, st, kStEmbBwd + 1);
  gather_and_reduce(M, st, nloc, ntarget, d_mapping, e, nloc, nullptr, out);
}

// complete: the list holds every neighbour within rcut of every centre and
// maps onto local owners (the standalone path), which the DPA4C fused force
// pass relies on
void run_model(dp_model* M, hipStream_t st, int nloc, int nall, const int* d_mapping, int ntarget,
               const Outputs& out, bool complete) {
  if (M->kind == dp_model::kDpa4c)
    return run_c4(M, st, nloc, d_mapping, ntarget, out, complete && d_mapping && ntarget == nloc);
  // the standalone path counts its ghosts on the device
  const int* d_nall = complete ? static_cast<const int*>(M->nall_d.p) : nullptr;
  if (M->precision == DP_PREC_MIXED)
    run_model_t<float>(M, st, nloc, nall, d_nall, d_mapping, ntarget, out);
  else
    run_model_t<double>(M, st, nloc, nall, d_nall, d_mapping, ntarget, out);
}

// Neighbour-list parameters of the model. DPA4C keeps r^2 < rcut^2 (strict,
// deepmd-op/overlays/op/pt/dpa4c/exact_cut.cuh:10-20) and never drops a
// neighbour: a section that overflows its capacity is an error.
NlParams nl_params(const dp_model* M) {
  const ModelHost& m = M->host;
  NlParams np{};
  np.ntypes = m.ntypes;
  np.nnei = m.nnei;
  for (int t = 0; t < m.ntypes; ++t) np.sel[t] = m.sel[t];
  for (int t = 0; t <= m.ntypes; ++t) np.sec[t] = m.sec[t];
  np.rc2 = m.rcut * m.rcut;
  if (M->kind == dp_model::kDpa4c) {
    np.rc2 = std::nextafter(np.rc2, 0.0);
    np.sel_strict = 1;
  }
  return np;
}

// DPA4C sums over a centre's edges in list order, which need not be by
// distance, only reproducible: the standalone list keeps candidate order over
// cell-ordered atoms (no rank pass). The LAMMPS list, whose candidate order is
// the caller's, stays sorted.
NlParams nl_params_cells(const dp_model* M) {
  NlParams np = nl_params(M);
  np.unsorted = M->kind == dp_model::kDpa4c ? 1 : 0;
  return np;
}

// Ghosts + cells + nlist for the standalone path, with no host round trip:
// the extended arrays are sized for every ghost candidate (nshift images of
// each local atom, the most the box can produce), the number of ghosts is
// counted on the device into nall_d, and the kernels over the extended atoms
// read it from there. Returns the capacity nall_cap (>= nall).
int build_standalone_nlist(dp_model* M, hipStream_t st, int nloc, const double* d_coord,
                           const int* d_atype, const BoxParams& bp) {
  const ModelHost& m = M->host;
  const long nf = bp.nshift > 0 ? (long)bp.nshift * nloc : 0;
  if (nloc + nf >= (1L << 31) - 1) throw ApiError{DP_ERR_CAPACITY, "too many ghost candidates"};
  const int nall_cap = nloc + (int)nf;
  const NlParams np = nl_params_cells(M);
  double* sfrac = need<double>(M, M->sfrac, (size_t)nloc * 3);
  double* ext = need<double>(M, M->ext, (size_t)nall_cap * 3);
  int* ext_type = need<int>(M, M->ext_type, (size_t)nall_cap);
  int* mapping = need<int>(M, M->mapping, (size_t)nall_cap);
  int* nall_d = need<int>(M, M->nall_d, 1);
  const int nall = nall_cap;
  const int ncell = bp.ncell[0] * bp.ncell[1] * bp.ncell[2];
  int* cell_of = need<int>(M, M->cell_of, (size_t)nall);
  int* ccount = need<int>(M, M->cell_count, (size_t)ncell + 1);
  int* cstart = need<int>(M, M->cell_start, (size_t)ncell + 1);
  int* crank = need<int>(M, M->cell_rank, (size_t)nall);
  CellAtom* sorted = need<CellAtom>(M, M->sorted, (size_t)nall);
  // the wrap also clears the cell counts (and gives nall when there are no
  // ghosts); the ghost placement gives nall otherwise
  launch_wrap(st, nloc, d_coord, d_atype, bp, ext, ext_type, mapping, sfrac, ncell + 1, ccount,
              nf > 0 ? nullptr : nall_d);
  if (nf > 0) {
    const long nc = (long)bp.nshift * ghost_tiles(nloc);  // per (shift, tile of atoms)
    int* count = need<int>(M, M->flags, (size_t)nc);
    int* first = need<int>(M, M->gpos, (size_t)nc);
    launch_ghost_count(st, nloc, bp, sfrac, count);
    const size_t tb = scan_temp_bytes((int)nc);
    void* tmp = need<char>(M, M->scan_tmp, tb);
    exclusive_scan_int(st, count, first, (int)nc, tmp, tb);
    launch_ghost_place(st, nloc, bp, sfrac, count, first, ext, ext_type, mapping, nall_d);
  }
  // cells
  launch_cell_assign(st, nall, nall_d, bp, ext, cell_of, crank, ccount);
  {
    const size_t tb = scan_temp_bytes(ncell + 1);
    void* tmp = need<char>(M, M->scan_tmp, tb);
    exclusive_scan_int(st, ccount, cstart, ncell + 1, tmp, tb);
  }
  launch_cell_scatter(st, nall, nall_d, cell_of, crank, cstart, ext, ext_type, sorted);
  if (np.unsorted) launch_cell_order(st, ncell, cstart, sorted);
  record(M, st, kStGeom + 1);
  int* nlist = need<int>(M, M->nlist, (size_t)std::max(nloc, 1) * m.nnei);
  int* nreal = need<int>(M, M->nreal, (size_t)std::max(nloc, 1) * m.ntypes);
  launch_nlist_cells(st, nloc, bp, np, ext, ext_type, cell_of, cstart, sorted, nall, nlist, nreal,
                     static_cast<int*>(M->status.p));
  record(M, st, kStNlist + 1);
  return nall;
}

void throw_status(int s) {
  if (s & kStatusNeighbourOverflow)
    throw ApiError{DP_ERR_CAPACITY, "more than " + std::to_string(kMaxCand) +
                                        " neighbours within rcut of one atom"};
  if (s & kStatusReverseOverflow)
    throw ApiError{DP_ERR_CAPACITY,
                   "more than " + std::to_string(kMaxRev) + " edges point at one atom"};
  if (s & kStatusSelOverflow)
    throw ApiError{DP_ERR_CAPACITY,
                   "more neighbours of one type within rcut than the model's sel holds"};
  if (s & kStatusBadInput)
    throw ApiError{DP_ERR_ARG, "atom type or edge source outside the model / graph"};
  if (s & kStatusFixedRange)
    throw ApiError{DP_ERR_CAPACITY,
                   "an edge's force is outside the fixed-point force accumulators' range "
                   "(|dE/dd| > " + std::to_string((int)kFixTermMax) +
                       " eV/A / max(1, rcut), or not finite)"};
}

void check_status(dp_model* M, hipStream_t st) {
  int s = 0;
  DPAMD_HIP(hipMemcpyAsync(&s, M->status.p, 4, hipMemcpyDeviceToHost, st));
  DPAMD_HIP(hipStreamSynchronize(st));
  throw_status(s);
}

// Adds the stage times of the oldest pending event set (waiting for it).
void harvest_oldest(dp_model* M) {
  const int k = (M->ev_head - M->ev_pending + dp_model::kRing) % dp_model::kRing;
  DPAMD_HIP(hipEventSynchronize(M->ev[k][kNumStages]));
  for (int q = 0; q < kNumStages; ++q) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, M->ev[k][q], M->ev[k][q + 1]) != hipSuccess) ms = 0.f;
    M->st_sum[q] += ms;
  }
  ++M->st_count;
  --M->ev_pending;
}

// Stage times = mean over the evaluations since the previous call.
void stage_times_of_last(dp_model* M) {
  if (!M->timing) return;
  while (M->ev_pending > 0) harvest_oldest(M);
  if (M->st_count == 0) return;
  for (int q = 0; q < kNumStages; ++q) {
    M->stage_ms[q] = (float)(M->st_sum[q] / M->st_count);
    M->st_sum[q] = 0.0;
  }
  M->st_count = 0;
}

// Waits for the evaluations queued by dp_compute_device_async and reports a
// capacity error any of them raised (clearing it).
void settle_async(dp_model* M) {
  if (!M->async_pending) return;
  M->async_pending = false;
  DPAMD_HIP(hipStreamSynchronize(M->async_stream));
  int s = 0;
  DPAMD_HIP(hipMemcpy(&s, M->status.p, 4, hipMemcpyDeviceToHost));
  stage_times_of_last(M);
  if (s) {
    // replayed graphs never clear the word themselves
    launch_fill_int(M->async_stream, 1, 0, static_cast<int*>(M->status.p));
    DPAMD_HIP(hipStreamSynchronize(M->async_stream));
    *M->status_host = 0;
    throw_status(s);
  }
}

// async: the status word is cleared only by the first evaluation after a
// settle, so a flag raised by any queued evaluation survives until read
void begin(dp_model* M, hipStream_t st, bool async = false) {
  DPAMD_HIP(hipSetDevice(M->device));
  if (!async) settle_async(M);
  int* status = need<int>(M, M->status, 1);
  if (!async || !M->async_pending) launch_fill_int(st, 1, 0, status);
  if (M->timing) {
    if (M->ev_pending == dp_model::kRing) harvest_oldest(M);
    M->ev_cur = M->ev_head;
    M->ev_head = (M->ev_head + 1) % dp_model::kRing;
    ++M->ev_pending;
    for (int q = 0; q <= kNumStages; ++q)
      if (!M->ev[M->ev_cur][q]) DPAMD_HIP(hipEventCreate(&M->ev[M->ev_cur][q]));
    DPAMD_HIP(hipEventRecord(M->ev[M->ev_cur][0], st));
  }
}

void finish(dp_model* M, hipStream_t st) {
  check_status(M, st);
  stage_times_of_last(M);
}

template <class F>
int guarded(dp_model* M, F&& f) {
  if (!M) return DP_ERR_ARG;
  try {
    M->err.clear();
    f();
    return DP_OK;
  } catch (const ApiError& e) {
    M->err = e.msg;
    return e.code;
  } catch (const HipError& e) {
    M->err = std::string("HIP error ") + hipGetErrorString(e.code) + " in " + e.where;
    return DP_ERR_HIP;
  } catch (const std::exception& e) {
    M->err = e.what();
    return DP_ERR_ARG;
  }
}

void graph_reset(dp_model* M) {
  if (M->graph_exec) (void)hipGraphExecDestroy(M->graph_exec);
  if (M->graph) (void)hipGraphDestroy(M->graph);
  M->graph_exec = nullptr;
  M->graph = nullptr;
}

// Runs the queued evaluation `body` as a graph replay (capturing it first
// when the key is new and one eager evaluation with that key has sized every
// buffer). Returns false when the caller must run it eagerly: the first call
// with a key, or after a failed capture (graphs are then off for the handle).
// The graph lives on a stream of its own: it waits for `st` on entry and
// `st` waits for it on exit, as the reference's replay does
// (DeepPotPTExpt.cc:122-191).
template <class Body>
bool graph_step(dp_model* M, hipStream_t st, int natoms, const double* d_coord,
                const int* d_atype, const double* box, const Outputs& o, Body&& body) {
  std::vector<unsigned char> key;
  auto put = [&](const void* p, size_t n) {
    const auto* b = static_cast<const unsigned char*>(p);
    key.insert(key.end(), b, b + n);
  };
  const void* ptrs[8] = {d_coord, d_atype, o.energy, o.force, o.virial, o.atom_energy,
                         o.atom_virial, st};
  put(&natoms, sizeof natoms);
  put(ptrs, sizeof ptrs);
  put(box, 9 * sizeof(double));
  put(&M->buf_gen, sizeof M->buf_gen);
  put(&M->bucket_gen, sizeof M->bucket_gen);
  if (key != M->graph_key) {
    graph_reset(M);
    M->graph_key = key;
    M->graph_warm = 0;
  }
  if (!M->graph_exec && M->graph_warm < 1) {
    ++M->graph_warm;  // eager run with this key first
    return false;
  }
  DPAMD_HIP(hipSetDevice(M->device));
  if (!M->graph_st) {
    DPAMD_HIP(hipStreamCreateWithFlags(&M->graph_st, hipStreamNonBlocking));
    DPAMD_HIP(hipEventCreateWithFlags(&M->graph_in, hipEventDisableTiming));
    DPAMD_HIP(hipEventCreateWithFlags(&M->graph_out, hipEventDisableTiming));
  }
  DPAMD_HIP(hipEventRecord(M->graph_in, st));
  DPAMD_HIP(hipStreamWaitEvent(M->graph_st, M->graph_in, 0));
  if (!M->graph_exec) {
    const unsigned long gen = M->buf_gen;
    bool ok = hipStreamBeginCapture(M->graph_st, hipStreamCaptureModeRelaxed) == hipSuccess;
    if (ok) {
      try {
        body(M->graph_st);
      } catch (...) {
        ok = false;
      }
      hipGraph_t g = nullptr;
      ok = hipStreamEndCapture(M->graph_st, &g) == hipSuccess && ok && g;
      // a buffer reallocated while capturing would leave stale pointers
      ok = ok && M->buf_gen == gen;
      if (ok) ok = hipGraphInstantiate(&M->graph_exec, g, nullptr, nullptr, 0) == hipSuccess;
      if (ok) M->graph = g;
      else if (g) (void)hipGraphDestroy(g);
    }
    if (!ok) {
      (void)hipGetLastError();
      graph_reset(M);
      M->graph_broken = true;
      // nothing was enqueued by the failed capture: run eagerly after all
      DPAMD_HIP(hipEventRecord(M->graph_out, M->graph_st));
      DPAMD_HIP(hipStreamWaitEvent(st, M->graph_out, 0));
      return false;
    }
    ++M->graph_captures;
  }
  DPAMD_HIP(hipGraphLaunch(M->graph_exec, M->graph_st));
  ++M->graph_replays;
  DPAMD_HIP(hipEventRecord(M->graph_out, M->graph_st));
  DPAMD_HIP(hipStreamWaitEvent(st, M->graph_out, 0));
  return true;
}

// One standalone evaluation on device buffers (dp_compute_device and its
// asynchronous form). async: no host synchronisation unless the type buckets
// must be rebuilt, and the status word is copied to pinned memory instead of
// being checked.
void device_step(dp_model* M, int natoms, const double* d_coord, const int* d_atype,
                 const double* box, int ago, double* d_energy, double* d_force, double* d_virial,
                 double* d_atom_energy, double* d_atom_virial, hipStream_t st, bool async) {
  if (natoms < 0 || (natoms > 0 && (!d_coord || !d_atype || !d_force)))
    throw ApiError{DP_ERR_ARG, "null device pointer"};
  if (!box) throw ApiError{DP_ERR_ARG, "dp_compute_device needs a periodic box"};
  if (async) {
    DPAMD_HIP(hipSetDevice(M->device));
    if (!M->status_host) {
      DPAMD_HIP(hipHostMalloc(reinterpret_cast<void**>(&M->status_host), 64, hipHostMallocDefault));
      *M->status_host = 0;
    }
    // a flag raised by an earlier queued evaluation that has landed already
    if (M->async_pending && *static_cast<volatile int*>(M->status_host)) settle_async(M);
    if (M->async_pending && M->async_stream != st) settle_async(M);
  }
  if (ago == 0 || !M->buckets_valid || (int)M->atype_cache.size() != natoms) {
    DPAMD_HIP(hipSetDevice(M->device));
    std::vector<int> at(natoms);
    if (natoms)
      DPAMD_HIP(hipMemcpyAsync(at.data(), d_atype, sizeof(int) * natoms, hipMemcpyDeviceToHost, st));
    DPAMD_HIP(hipStreamSynchronize(st));
    M->buckets_valid = false;
    update_buckets(M, natoms, at.data(), st);
  }
  const BoxParams bp = make_box(box, M->host.rcut);
  Outputs o{d_energy, d_force, d_virial, d_atom_energy, d_atom_virial};
  // the evaluation proper: no host synchronisation, no allocation once sized
  auto body = [&](hipStream_t s) {
    const int nall = build_standalone_nlist(M, s, natoms, d_coord, d_atype, bp);
    run_model(M, s, natoms, nall, static_cast<const int*>(M->mapping.p), natoms, o, true);
    if (async) DPAMD_HIP(hipMemcpyAsync(M->status_host, M->status.p, 4, hipMemcpyDeviceToHost, s));
    M->last_nall = nall;
  };
  M->last_nloc = natoms;
  M->last_standalone = true;
  const bool try_graph = async && M->graph_on && !M->graph_broken && !M->timing && natoms > 0;
  if (try_graph && !M->async_pending) {
    // a graph does not clear the status word: start the queue from zero
    DPAMD_HIP(hipSetDevice(M->device));
    launch_fill_int(st, 1, 0, need<int>(M, M->status, 1));
  }
  if (try_graph && graph_step(M, st, natoms, d_coord, d_atype, box, o, body)) {
    M->async_stream = st;
    M->async_pending = true;
    return;
  }
  begin(M, st, async);
  body(st);
  if (async) {
    M->async_stream = st;
    M->async_pending = true;
  } else {
    finish(M, st);
  }
}

// se_e2_a groups centres by type on the host: the edge entry points carry no
// `ago`, so the local types are read back on every call (nloc ints) and the
// grouping is rebuilt only when they changed. DPA4C needs no grouping.
void edges_types(dp_model* M, const int* d_atype, int nloc, hipStream_t st) {
  if (M->kind != dp_model::kSeA) return;
  DPAMD_HIP(hipSetDevice(M->device));
  settle_async(M);
  std::vector<int> at(std::max(nloc, 0));
  if (nloc > 0) {
    if (!d_atype) throw ApiError{DP_ERR_ARG, "null device pointer"};
    DPAMD_HIP(hipMemcpyAsync(at.data(), d_atype, sizeof(int) * nloc, hipMemcpyDeviceToHost, st));
  }
  DPAMD_HIP(hipStreamSynchronize(st));
  update_buckets(M, nloc, at.data(), st);
}

// The compute_edges_gpu path (dp_compute_edges_device*): the caller's edge
// graph becomes extended atoms (edges.hip), its candidate CSR by centre is
// sel-formatted by the LAMMPS-list kernel, and the model runs with forces
// gathered onto the edges' source nodes.
template <class T>
void edges_step(dp_model* M, double* d_atom_energy, double* d_force, double* d_atom_virial,
                const int* d_atype, const int* d_edge_index, const T* d_edge_vec, int nloc,
                int nedge, int nall_nodes, hipStream_t st) {
  const int nnode = nall_nodes > 0 ? nall_nodes : nloc;
  if (nloc < 0 || nedge < 0 || nnode < nloc)
    throw ApiError{DP_ERR_ARG, "invalid edge graph dimensions"};
  if ((nnode > 0 && (!d_atype || !d_force || !d_atom_virial)) ||
      (nedge > 0 && (!d_edge_index || !d_edge_vec)) || (nloc > 0 && !d_atom_energy))
    throw ApiError{DP_ERR_ARG, "null device pointer"};
  if ((long)nloc + nedge >= (1L << 31) - 1) throw ApiError{DP_ERR_CAPACITY, "too many edges"};
  begin(M, st);
  const ModelHost& m = M->host;
  int* status = static_cast<int*>(M->status.p);
  const int nall = nloc + nedge;
  double* ext = need<double>(M, M->ext, (size_t)std::max(nall, 1) * 3);
  int* ext_type = need<int>(M, M->ext_type, (size_t)std::max(nall, 1));
  int* mapping = need<int>(M, M->mapping, (size_t)std::max(nall, 1));
  int* count = need<int>(M, M->cell_count, (size_t)nloc + 1);
  int* off = need<int>(M, M->cell_start, (size_t)nloc + 1);
  int* rank = need<int>(M, M->cell_rank, (size_t)std::max(nedge, 1));
  long* cand_off = need<long>(M, M->cand_off, (size_t)nloc + 1);
  int* cand = need<int>(M, M->cand, (size_t)std::max(nedge, 1));
  // the edge graph's candidates overwrite a cached LAMMPS list
  M->cand_valid = false;
  launch_fill_int(st, (long)nloc + 1, 0, count);
  launch_edges_ext<T>(st, nloc, nedge, nnode, d_edge_index, d_edge_vec, d_atype, ext, ext_type,
                      mapping, count, rank, status);
  {
    const size_t tb = scan_temp_bytes(nloc + 1);
    void* tmp = need<char>(M, M->scan_tmp, tb);
    exclusive_scan_int(st, count, off, nloc + 1, tmp, tb);
  }
  launch_edges_fill(st, nloc, nedge, nnode, d_edge_index, off, rank, cand_off, cand);
  record(M, st, kStGeom + 1);
  const NlParams np = nl_params(M);
  int* nlist = need<int>(M, M->nlist, (size_t)std::max(nloc, 1) * m.nnei);
  int* nreal = need<int>(M, M->nreal, (size_t)std::max(nloc, 1) * m.ntypes);
  launch_nlist_csr(st, nloc, np, ext, ext_type, cand_off, cand, nlist, nreal, status);
  record(M, st, kStNlist + 1);
  // atom energies go through a workspace over every node (the gather zeroes
  // ntarget of them), of which the first nloc are the caller's
  double* ae = need<double>(M, M->ae_ws, (size_t)std::max(nnode, 1));
  Outputs o{nullptr, d_force, nullptr, ae, d_atom_virial};
  run_model(M, st, nloc, nall, mapping, nnode, o, false);
  if (nloc > 0)
    DPAMD_HIP(hipMemcpyAsync(d_atom_energy, ae, sizeof(double) * nloc, hipMemcpyDeviceToDevice, st));
  M->last_nloc = nloc;
  M->last_nall = nall;
  M->last_standalone = false;
  finish(M, st);
}

// Packs every DPA4C parameter array into one device allocation (each array
// 256-byte aligned) and points the kernel parameters at it.
void upload_c4(dp_model* M) {
  const C4Host& c = M->c4;
  const ModelHost& m = M->host;
  std::vector<unsigned char> blob;
  auto put = [&](const void* src, size_t bytes) {
    const size_t off = (blob.size() + 255) & ~size_t(255);
    blob.resize(off + bytes);
    std::memcpy(blob.data() + off, src, bytes);
    return off;
  };
  const size_t o_table = put(c.table.data(), c.table.size() * 4);
  const size_t o_film = put(c.film.data(), c.film.size() * 4);
  const size_t o_ro = put(c.ro.data(), c.ro.size() * 4);
  const size_t o_temb = put(c.temb.data(), c.temb.size() * 4);
  const size_t o_mean = put(c.mean.data(), c.mean.size() * 4);
  const size_t o_istd = put(c.istd.data(), c.istd.size() * 4);
  const size_t o_w0t = put(c.w0t.data(), c.w0t.size() * 4);
  const size_t o_b0 = put(c.b0.data(), c.b0.size() * 4);
  const size_t o_wh = put(c.wh.data(), c.wh.size() * 4);
  const size_t o_bias = put(c.bias.data(), c.bias.size() * 8);
  DPAMD_HIP(hipMalloc(&M->d_c4, blob.size()));
  M->bytes_now += blob.size();
  M->bytes_peak = std::max(M->bytes_peak, M->bytes_now);
  DPAMD_HIP(hipMemcpy(M->d_c4, blob.data(), blob.size(), hipMemcpyHostToDevice));
  const auto* base = static_cast<const unsigned char*>(M->d_c4);
  C4Params& p = M->c4p;
  p.table = reinterpret_cast<const float*>(base + o_table);
  p.film = reinterpret_cast<const float*>(base + o_film);
  p.ro = reinterpret_cast<const float*>(base + o_ro);
  p.temb = reinterpret_cast<const float*>(base + o_temb);
  p.mean = reinterpret_cast<const float*>(base + o_mean);
  p.istd = reinterpret_cast<const float*>(base + o_istd);
  p.w0t = reinterpret_cast<const float*>(base + o_w0t);
  p.b0 = reinterpret_cast<const float*>(base + o_b0);
  p.wh = reinterpret_cast<const float*>(base + o_wh);
  p.bias = reinterpret_cast<const double*>(base + o_bias);
  p.bh = c.bh;
  p.nt = m.ntypes;
  p.n_int = c.n_int;
  p.H = c.H;
  p.act = c.act;
  p.resnet = c.resnet;
  p.rcut = (float)m.rcut;
  p.inv_rcut = (float)(1.0 / m.rcut);
  p.eps2 = (float)(c.eps * c.eps);
  p.floor = (float)c.floor;
  p.stride = (float)c.stride;
  p.inv_stride = (float)(1.0 / c.stride);
  p.ncu = M->ncu;
}

}  // namespace

extern "C" {

int dp_create(const char* path, int gpu_rank, const void* file_content, size_t content_len,
              int precision, dp_model** out) {
  if (!out) return DP_ERR_ARG;
  *out = nullptr;
  dp_model* M = new dp_model();
  int rc = guarded(M, [&]() {
    if (precision != DP_PREC_FP64 && precision != DP_PREC_MIXED && precision != DP_PREC_MODEL)
      throw ApiError{DP_ERR_ARG, "precision must be DP_PREC_MODEL, DP_PREC_FP64 or DP_PREC_MIXED"};
    std::vector<unsigned char> buf;
    if (file_content && content_len) {
      const auto* b = static_cast<const unsigned char*>(file_content);
      buf.assign(b, b + content_len);
    } else {
      if (!path) throw ApiError{DP_ERR_ARG, "no model path or content"};
      std::ifstream f(path, std::ios::binary);
      if (!f) throw ApiError{DP_ERR_MODEL, std::string("cannot open model file ") + path};
      buf.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    }
    const bool c4 = buf.size() >= 8 && std::memcmp(buf.data(), "DPAMDC4N", 8) == 0;
    M->kind = c4 ? dp_model::kDpa4c : dp_model::kSeA;
    const std::string perr = c4 ? parse_c4_model(buf.data(), buf.size(), M->host, M->c4)
                                : parse_model(buf.data(), buf.size(), M->host);
    if (!perr.empty()) throw ApiError{DP_ERR_MODEL, perr};
    if (precision == DP_PREC_MODEL) precision = M->host.precision;
    M->precision = precision;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
      throw ApiError{DP_ERR_NO_GPU, "no HIP device visible"};
    if (gpu_rank < 0) gpu_rank = 0;
    M->device = gpu_rank % ndev;
    DPAMD_HIP(hipSetDevice(M->device));
    hipDeviceProp_t prop;
    DPAMD_HIP(hipGetDeviceProperties(&prop, M->device));
    M->ncu = std::max(1, prop.multiProcessorCount);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      throw ApiError{DP_ERR_NO_GPU, std::string("device is ") + prop.gcnArchName +
                                        ", this library is built for gfx950"};
    // the device's static scratch of the no-allocation entry point (its
    // address, looked up once per device)
    M->arena_base = static_cast<char*>(noalloc_scratch_init(M->device));
    if (c4) {
      // DPA4C nets are fp32 by definition (fp64 energies, forces and virials)
      M->precision = DP_PREC_MIXED;
      upload_c4(M);
      return;
    }
    const ModelHost& m = M->host;
    const bool mixed = precision == DP_PREC_MIXED;
    M->el = make_emb_layout(m.emb[0], m.emb[1], m.emb[2], mixed);
    std::vector<double> emb, envp, tpad;
    pack_embedding(m, M->el, emb, envp, tpad);
    auto upload = [&](auto*& dst, const auto& src) {
      const size_t bytes = src.size() * sizeof(src[0]);
      void* p = nullptr;
      DPAMD_HIP(hipMalloc(&p, std::max<size_t>(8, bytes)));
      dst = static_cast<std::remove_reference_t<decltype(dst)>>(p);
      M->bytes_now += bytes;
      DPAMD_HIP(hipMemcpy(p, src.data(), bytes, hipMemcpyHostToDevice));
    };
    upload(M->d_envp, envp);
    upload(M->d_tpad, tpad);
    if (mixed) {
      // the nets are evaluated in fp32: round the parameters once here
      std::vector<float> emb32(emb.begin(), emb.end());
      pack_embedding_bf16(m, M->el, emb32);
      const std::vector<float> fit32(m.fit_params.begin(), m.fit_params.end());
      upload(M->d_emb, emb32);
      upload(M->d_fit, fit32);
      // fitting GEMM operands pre-split for the bf16 matrix cores: W0, W1,
      // W2 forward, W1 / W2 transposed, and W0 transposed tile-major for the
      // fused dE/dD -> dE/dT kernel (when it applies; otherwise dE/dD is
      // the plain fp32 product of the library's GEMM, then the dE/dT pass)
      const FitOffsets fo = fit_offsets(m);
      const int ins[3] = {m.emb[2] * m.axis, m.fit[0], m.fit[1]};
      const bool w0t = ddt_supported(m.fit[0], m.emb[2], m.axis);
      std::vector<uint16_t> frag;
      for (int t = 0; t < m.ntypes; ++t)
        for (int k = 0; k < 3; ++k)
          for (int tr = 0; tr < 2; ++tr) {
            M->fitf_off[t][k][tr] = -1;
            if (k == 0 && tr == 1 && !w0t) continue;
            frag.resize((frag.size() + 127) / 128 * 128);  // 256-byte aligned blocks
            M->fitf_off[t][k][tr] = (long)(frag.size() * sizeof(uint16_t));
            pack_gemm_bf16(m.fit_params.data() + (size_t)t * m.fit_block + fo.W[k], ins[k],
                           m.fit[k], tr == 1, frag, k == 0 && tr == 1);
          }
      upload(M->d_fitf, frag);
    } else {
      upload(M->d_emb, emb);
      upload(M->d_fit, m.fit_params);
      const int Dn = m.emb[2] * m.axis, F0 = m.fit[0];
      if (ddt_supported(F0, m.emb[2], m.axis)) {
        const FitOffsets fo = fit_offsets(m);
        std::vector<double> w0t((size_t)m.ntypes * F0 * Dn);
        for (int t = 0; t < m.ntypes; ++t) {
          const double* W = m.fit_params.data() + (size_t)t * m.fit_block + fo.W[0];
          for (int n = 0; n < Dn; ++n)
            for (int k = 0; k < F0; ++k) w0t[((size_t)t * F0 + k) * Dn + n] = W[(size_t)n * F0 + k];
        }
        upload(M->d_w0t, w0t);
      }
    }
    M->bytes_peak = M->bytes_now;
    M->fo = fit_offsets(m);
    if (const char* g = std::getenv("DPAMD_GRAPH")) M->graph_on = std::atoi(g) != 0;
  });
  if (rc != DP_OK) {
    // keep the handle so the caller can read dp_last_error, unless nothing usable
    *out = M;
    return rc;
  }
  *out = M;
  return DP_OK;
}

void dp_destroy(dp_model* M) {
  if (!M) return;
  // teardown is best effort: errors here have nowhere to go
  (void)hipSetDevice(M->device);
  for (Buf* b : M->bufs)
    if (b->p) (void)hipFree(b->p);
  for (void* p : {M->d_emb, static_cast<void*>(M->d_envp), static_cast<void*>(M->d_tpad), M->d_fit,
                  M->d_fitf, M->d_c4, static_cast<void*>(M->d_w0t)})
    if (p) (void)hipFree(p);
  if (M->async_pending) (void)hipStreamSynchronize(M->async_stream);
  for (auto& set : M->ev)
    for (hipEvent_t e : set)
      if (e) (void)hipEventDestroy(e);
  if (M->status_host) (void)hipHostFree(M->status_host);
  for (int t = 0; t < kMaxTypes; ++t) {
    if (M->fit_st[t]) (void)hipStreamDestroy(M->fit_st[t]);
    if (M->join_ev[t]) (void)hipEventDestroy(M->join_ev[t]);
  }
  if (M->fork_ev) (void)hipEventDestroy(M->fork_ev);
  graph_reset(M);
  if (M->graph_st) (void)hipStreamDestroy(M->graph_st);
  if (M->graph_in) (void)hipEventDestroy(M->graph_in);
  if (M->graph_out) (void)hipEventDestroy(M->graph_out);
  delete M;
}

int dp_get_info(const dp_model* M, dp_model_info* info) {
  if (!M || !info) return DP_ERR_ARG;
  std::memset(info, 0, sizeof(*info));
  const ModelHost& m = M->host;
  info->ntypes = m.ntypes;
  info->nnei = m.nnei;
  for (int t = 0; t < m.ntypes; ++t) {
    info->sel[t] = m.sel[t];
    std::strncpy(info->type_map[t], m.type_map[t].c_str(), 15);
  }
  info->rcut = m.rcut;
  info->rcut_smth = m.rcut_smth;
  for (int k = 0; k < 3; ++k) {
    info->emb[k] = m.emb[k];
    info->fit[k] = m.fit[k];
  }
  info->axis = m.axis;
  info->precision = M->precision;
  info->model_kind = M->kind == dp_model::kDpa4c ? DP_MODEL_DPA4C : DP_MODEL_SE_E2_A;
  if (M->kind == dp_model::kDpa4c) {
    // channel widths C0, C1, C2 and the hidden width of the fitting net
    info->emb[0] = 8;
    info->emb[1] = 4;
    info->emb[2] = 4;
    info->fit[0] = M->c4.H;
  }
  return DP_OK;
}

const char* dp_last_error(const dp_model* M) { return M ? M->err.c_str() : "null handle"; }

int dp_compute_device(dp_model* M, int natoms, const double* d_coord, const int* d_atype,
                      const double* box, int ago, double* d_energy, double* d_force,
                      double* d_virial, double* d_atom_energy, double* d_atom_virial,
                      void* stream) {
  return guarded(M, [&]() {
    device_step(M, natoms, d_coord, d_atype, box, ago, d_energy, d_force, d_virial, d_atom_energy,
                d_atom_virial, static_cast<hipStream_t>(stream), false);
  });
}

int dp_compute_device_async(dp_model* M, int natoms, const double* d_coord, const int* d_atype,
                            const double* box, int ago, double* d_energy, double* d_force,
                            double* d_virial, double* d_atom_energy, double* d_atom_virial,
                            void* stream) {
  return guarded(M, [&]() {
    device_step(M, natoms, d_coord, d_atype, box, ago, d_energy, d_force, d_virial, d_atom_energy,
                d_atom_virial, static_cast<hipStream_t>(stream), true);
  });
}

// The evaluation of dp_compute_device with every buffer carved from the
// device's static scratch: the handle's own buffers are set aside for the
// call and restored after it, and the state that refers to buffer contents
// (type buckets, stage copies) is invalidated, since the scratch is shared by
// every handle on the device.
int dp_compute_device_noalloc(dp_model* M, int natoms, const double* d_coord, const int* d_atype,
                              const double* box, double* d_energy, double* d_force,
                              double* d_virial, double* d_atom_energy, double* d_atom_virial,
                              void* stream) {
  return guarded(M, [&]() {
    DPAMD_HIP(hipSetDevice(M->device));
    {
      // the call synchronises and reads back from the host: it cannot be
      // recorded into a graph, and trying would invalidate the capture
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      DPAMD_HIP(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs));
      if (cs != hipStreamCaptureStatusNone)
        throw ApiError{DP_ERR_ARG,
                       "dp_compute_device_noalloc is synchronous and cannot run on a stream "
                       "under graph capture"};
    }
    settle_async(M);
    if (!M->arena_base) throw ApiError{DP_ERR_NO_GPU, "no static scratch on this device"};
    // every handle on the device carves from the same scratch: one call at
    // a time, from the first carve to the restore
    std::lock_guard<std::mutex> lock(noalloc_device_mutex(M->device));
    std::vector<Buf> saved;
    saved.reserve(M->bufs.size());
    for (Buf* b : M->bufs) {
      saved.push_back(*b);
      *b = Buf{};
    }
    const bool timing = M->timing;
    M->timing = false;
    M->arena_on = true;
    M->arena_cap = noalloc_scratch_bytes();
    M->arena_used = 0;
    M->buckets_valid = false;
    auto restore = [&]() {
      for (size_t k = 0; k < M->bufs.size(); ++k) *M->bufs[k] = saved[k];
      M->arena_on = false;
      M->timing = timing;
      M->buckets_valid = false;
      M->last_nloc = 0;
      M->last_nall = 0;
      M->last_standalone = false;
      M->eg_valid = false;
      M->dd_valid = false;
    };
    try {
      device_step(M, natoms, d_coord, d_atype, box, 0, d_energy, d_force, d_virial, d_atom_energy,
                  d_atom_virial, static_cast<hipStream_t>(stream), false);
    } catch (...) {
      // kernels already queued only touch the scratch: let them finish
      (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));
      restore();
      throw;
    }
    restore();
  });
}

int dp_graph_stats(const dp_model* M, long* captures, long* replays) {
  if (!M) return DP_ERR_ARG;
  if (captures) *captures = M->graph_captures;
  if (replays) *replays = M->graph_replays;
  return M->graph_on && !M->graph_broken ? 1 : 0;
}

int dp_sync(dp_model* M) {
  return guarded(M, [&]() {
    DPAMD_HIP(hipSetDevice(M->device));
    settle_async(M);
  });
}

int dp_compute(dp_model* M, int natoms, const double* coord, const int* atype, const double* box,
               double* energy, double* force, double* virial, double* atom_energy,
               double* atom_virial) {
  return guarded(M, [&]() {
    if (natoms < 0 || (natoms > 0 && (!coord || !atype)))
      throw ApiError{DP_ERR_ARG, "null coord/atype"};
    hipStream_t st = nullptr;
    begin(M, st);
    update_buckets(M, natoms, atype, st);
    const BoxParams bp = box ? make_box(box, M->host.rcut)
                             : make_open_frame(natoms, coord, M->host.rcut);
    double* dc = need<double>(M, M->coord_in, (size_t)std::max(natoms, 1) * 3);
    int* da = need<int>(M, M->atype_in, (size_t)std::max(natoms, 1));
    if (natoms) {
      DPAMD_HIP(hipMemcpyAsync(dc, coord, sizeof(double) * 3 * natoms, hipMemcpyHostToDevice, st));
      DPAMD_HIP(hipMemcpyAsync(da, atype, sizeof(int) * natoms, hipMemcpyHostToDevice, st));
    }
    const int nall = build_standalone_nlist(M, st, natoms, dc, da, bp);
    double* f = need<double>(M, M->force_ws, (size_t)std::max(natoms, 1) * 3);
    double* av = atom_virial ? need<double>(M, M->av_ws, (size_t)std::max(natoms, 1) * 9) : nullptr;
    double* ae = atom_energy ? need<double>(M, M->ae_ws, (size_t)std::max(natoms, 1)) : nullptr;
    double* o10 = need<double>(M, M->out10, 10);
    Outputs o{nullptr, f, nullptr, ae, av};
    run_model(M, st, natoms, nall, static_cast<const int*>(M->mapping.p), natoms, o, true);
    M->last_nloc = natoms;
    M->last_nall = nall;
    M->last_standalone = true;
    finish(M, st);
    double ev[10];
    DPAMD_HIP(hipMemcpy(ev, o10, sizeof(ev), hipMemcpyDeviceToHost));
    if (energy) *energy = ev[0];
    if (virial) std::memcpy(virial, ev + 1, 72);
    if (force && natoms) DPAMD_HIP(hipMemcpy(force, f, sizeof(double) * 3 * natoms, hipMemcpyDeviceToHost));
    if (atom_energy && natoms)
      DPAMD_HIP(hipMemcpy(atom_energy, ae, sizeof(double) * natoms, hipMemcpyDeviceToHost));
    if (atom_virial && natoms)
      DPAMD_HIP(hipMemcpy(atom_virial, av, sizeof(double) * 9 * natoms, hipMemcpyDeviceToHost));
  });
}

int dp_compute_nlist(dp_model* M, int nall, int nghost, const double* coord, const int* atype,
                     const double* box, int inum, const int* ilist, const int* numneigh,
                     const int* const* firstneigh, int neigh_mask, int ago, double* energy,
                     double* force, double* virial, double* atom_energy, double* atom_virial) {
  return guarded(M, [&]() {
    (void)box;
    const int nloc = nall - nghost;
    if (nall < 0 || nghost < 0 || nloc < 0) throw ApiError{DP_ERR_ARG, "bad nall/nghost"};
    if (nall > 0 && (!coord || !atype)) throw ApiError{DP_ERR_ARG, "null coord/atype"};
    if (inum > 0 && (!ilist || !numneigh || !firstneigh))
      throw ApiError{DP_ERR_ARG, "null neighbour list"};
    hipStream_t st = nullptr;
    begin(M, st);
    const ModelHost& m = M->host;
    update_buckets(M, nloc, atype, st);
    double* ext = need<double>(M, M->ext, (size_t)std::max(nall, 1) * 3);
    int* ext_type = need<int>(M, M->ext_type, (size_t)std::max(nall, 1));
    if (nall) {
      DPAMD_HIP(hipMemcpyAsync(ext, coord, sizeof(double) * 3 * nall, hipMemcpyHostToDevice, st));
      DPAMD_HIP(hipMemcpyAsync(ext_type, atype, sizeof(int) * nall, hipMemcpyHostToDevice, st));
    }
    if (ago == 0 || !M->cand_valid || M->cand_nloc != nloc || M->cand_nall != nall) {
      std::vector<long> off(nloc + 1, 0);
      std::vector<int> cnt(nloc, 0);
      for (int ii = 0; ii < inum; ++ii) {
        const int i = ilist[ii];
        if (i < 0 || i >= nloc) throw ApiError{DP_ERR_ARG, "ilist entry outside local atoms"};
        cnt[i] = numneigh[ii];
      }
      for (int i = 0; i < nloc; ++i) off[i + 1] = off[i] + cnt[i];
      std::vector<int> cand(std::max<long>(off[nloc], 1));
      for (int ii = 0; ii < inum; ++ii) {
        const int i = ilist[ii];
        for (int q = 0; q < numneigh[ii]; ++q) {
          int j = firstneigh[ii][q];
          if (neigh_mask) j &= neigh_mask;
          if (j < 0 || j >= nall) throw ApiError{DP_ERR_ARG, "neighbour index outside nall"};
          cand[off[i] + q] = j;
        }
      }
      long* d_off = need<long>(M, M->cand_off, (size_t)nloc + 1);
      int* d_cand = need<int>(M, M->cand, cand.size());
      DPAMD_HIP(hipMemcpyAsync(d_off, off.data(), sizeof(long) * (nloc + 1), hipMemcpyHostToDevice, st));
      DPAMD_HIP(hipMemcpyAsync(d_cand, cand.data(), sizeof(int) * cand.size(), hipMemcpyHostToDevice, st));
      DPAMD_HIP(hipStreamSynchronize(st));
      M->cand_valid = true;
      M->cand_nloc = nloc;
      M->cand_nall = nall;
    }
    record(M, st, kStGeom + 1);
    const NlParams np = nl_params(M);
    int* nlist = need<int>(M, M->nlist, (size_t)std::max(nloc, 1) * m.nnei);
    int* nreal = need<int>(M, M->nreal, (size_t)std::max(nloc, 1) * m.ntypes);
    launch_nlist_csr(st, nloc, np, ext, ext_type, static_cast<const long*>(M->cand_off.p),
                     static_cast<const int*>(M->cand.p), nlist, nreal,
                     static_cast<int*>(M->status.p));
    record(M, st, kStNlist + 1);
    double* f = need<double>(M, M->force_ws, (size_t)std::max(nall, 1) * 3);
    double* av = atom_virial ? need<double>(M, M->av_ws, (size_t)std::max(nall, 1) * 9) : nullptr;
    double* ae = atom_energy ? need<double>(M, M->ae_ws, (size_t)std::max(nall, 1)) : nullptr;
    double* o10 = need<double>(M, M->out10, 10);
    Outputs o{nullptr, f, nullptr, ae, av};
    run_model(M, st, nloc, nall, nullptr, nall, o, false);
    M->last_nloc = nloc;
    M->last_nall = nall;
    M->last_standalone = false;
    finish(M, st);
    double ev[10];
    DPAMD_HIP(hipMemcpy(ev, o10, sizeof(ev), hipMemcpyDeviceToHost));
    if (energy) *energy = ev[0];
    if (virial) std::memcpy(virial, ev + 1, 72);
    if (force && nall) DPAMD_HIP(hipMemcpy(force, f, sizeof(double) * 3 * nall, hipMemcpyDeviceToHost));
    if (atom_energy && nall)
      DPAMD_HIP(hipMemcpy(atom_energy, ae, sizeof(double) * nall, hipMemcpyDeviceToHost));
    if (atom_virial && nall)
      DPAMD_HIP(hipMemcpy(atom_virial, av, sizeof(double) * 9 * nall, hipMemcpyDeviceToHost));
  });
}

int dp_compute_canonical_graph_device(dp_model* M, double* d_atom_energy, double* d_force,
                                      double* d_atom_virial, const int64_t* d_atype,
                                      const uint32_t* d_source, const float* d_edge_vec,
                                      const int64_t* d_destination_row_ptr,
                                      const int64_t* d_source_row_ptr,
                                      const uint32_t* d_source_order, int nloc, int nall_nodes,
                                      int64_t edge_storage, void* stream) {
  return guarded(M, [&]() {
    if (M->kind != dp_model::kDpa4c)
      throw ApiError{DP_ERR_MODEL, "compute_canonical_graph_gpu requires a DPA4C model"};
    if (nloc < 0 || nall_nodes <= 0 || nloc > nall_nodes || edge_storage < 2 ||
        (uint64_t)edge_storage > 0xffffffffull)
      throw ApiError{DP_ERR_ARG, "invalid compact canonical graph dimensions."};
    if (!d_atype || !d_source || !d_edge_vec || !d_destination_row_ptr || !d_source_row_ptr ||
        !d_source_order || !d_force || !d_atom_virial || (nloc > 0 && !d_atom_energy))
      throw ApiError{DP_ERR_ARG, "null device pointer"};
    hipStream_t st = static_cast<hipStream_t>(stream);
    begin(M, st);
    int* status = static_cast<int*>(M->status.p);
    C4Graph g{};
    g.row_ptr = reinterpret_cast<const long*>(d_destination_row_ptr);
    g.source = d_source;
    g.edge_vec = d_edge_vec;
    g.atype = reinterpret_cast<const long*>(d_atype);
    g.nall = nall_nodes;
    g.storage = edge_storage;
    g.status = status;
    float* mom = need<float>(M, M->c4_mom, (size_t)std::max(nloc, 1) * kC4Mom);
    float* cot = need<float>(M, M->c4_cot, (size_t)std::max(nloc, 1) * kC4Mom);
    double* eg = need<double>(M, M->edge_grad, (size_t)edge_storage * 3);
    record(M, st, kStNlist + 1);
    launch_c4_moments(st, M->c4p, g, nloc, mom, status);
    record(M, st, kStEmbFwd + 1);
    record(M, st, kStDescr + 1);
    launch_c4_node(st, M->c4p, nloc, g.atype, mom, d_atom_energy, cot);
    record(M, st, kStFit + 1);
    record(M, st, kStDT + 1);
    launch_c4_edge_grad(st, M->c4p, g, nloc, cot, eg);
    launch_c4_zero_tail(st, g.row_ptr, nloc, edge_storage, eg);
    M->eg_valid = true;
    record(M, st, kStEmbBwd + 1);
    launch_c4_graph_force(st, nall_nodes, g.row_ptr, reinterpret_cast<const long*>(d_source_row_ptr),
                          d_source_order, d_edge_vec, eg, edge_storage, d_force, d_atom_virial,
                          status);
    record(M, st, kStForce + 1);
    record(M, st, kStReduce + 1);
    M->last_nloc = nloc;
    M->last_nall = nall_nodes;
    M->last_standalone = false;
    finish(M, st);
  });
}

int dp_compute_edges_device(dp_model* M, double* d_atom_energy, double* d_force,
                            double* d_atom_virial, const double* d_coord, const int* d_atype,
                            const int* d_edge_index, const double* d_edge_vec, int nloc,
                            int nedge, int nall_nodes, void* stream) {
  (void)d_coord;
  return guarded(M, [&]() {
    edges_types(M, d_atype, nloc, static_cast<hipStream_t>(stream));
    edges_step<double>(M, d_atom_energy, d_force, d_atom_virial, d_atype, d_edge_index,
                       d_edge_vec, nloc, nedge, nall_nodes, static_cast<hipStream_t>(stream));
  });
}

int dp_compute_edges_device_f32(dp_model* M, double* d_atom_energy, double* d_force,
                                double* d_atom_virial, const double* d_coord, const int* d_atype,
                                const int* d_edge_index, const float* d_edge_vec, int nloc,
                                int nedge, int nall_nodes, void* stream) {
  (void)d_coord;
  return guarded(M, [&]() {
    edges_types(M, d_atype, nloc, static_cast<hipStream_t>(stream));
    edges_step<float>(M, d_atom_energy, d_force, d_atom_virial, d_atype, d_edge_index, d_edge_vec,
                      nloc, nedge, nall_nodes, static_cast<hipStream_t>(stream));
  });
}

long dp_debug_copy(dp_model* M, int stage, void* dst, size_t capacity) {
  if (!M) return DP_ERR_ARG;
  long result = 0;
  const int rc = guarded(M, [&]() {
    const ModelHost& m = M->host;
    const int nloc = M->last_nloc;
    int nall = M->last_nall;
    if (M->last_standalone && M->nall_d.p) {
      // the standalone path counts its ghosts on the device
      DPAMD_HIP(hipDeviceSynchronize());
      DPAMD_HIP(hipMemcpy(&nall, M->nall_d.p, sizeof(int), hipMemcpyDeviceToHost));
    }
    const int Dn = m.emb[2] * m.axis;
    const size_t net_esize = M->precision == DP_PREC_MIXED ? 4 : 8;
    auto copy = [&](const void* src, size_t bytes) {
      result = (long)bytes;
      if (dst && capacity && src) {
        DPAMD_HIP(hipDeviceSynchronize());
        DPAMD_HIP(hipMemcpy(dst, src, std::min(bytes, capacity), hipMemcpyDeviceToHost));
      }
    };
    // bucket-ordered arrays are returned in atom order, widened to fp64 when
    // the mode keeps them in fp32 (esize 4)
    auto copy_bucket = [&](const void* src, size_t per_atom, size_t esize) {
      const size_t bytes = (size_t)nloc * per_atom * sizeof(double);
      result = (long)bytes;
      if (!dst || !capacity || !src) return;
      std::vector<double> tmp((size_t)M->nbucket * per_atom);
      DPAMD_HIP(hipDeviceSynchronize());
      if (!tmp.empty() && esize == 8)
        DPAMD_HIP(hipMemcpy(tmp.data(), src, tmp.size() * 8, hipMemcpyDeviceToHost));
      if (!tmp.empty() && esize == 4) {
        std::vector<float> t32(tmp.size());
        DPAMD_HIP(hipMemcpy(t32.data(), src, t32.size() * 4, hipMemcpyDeviceToHost));
        std::copy(t32.begin(), t32.end(), tmp.begin());
      }
      std::vector<double> outv((size_t)nloc * per_atom, 0.0);
      for (int p = 0; p < M->nbucket; ++p)
        std::memcpy(&outv[(size_t)M->items_h[p] * per_atom], &tmp[(size_t)p * per_atom],
                    per_atom * 8);
      std::memcpy(dst, outv.data(), std::min(bytes, capacity));
    };
    switch (stage) {
      case DP_STAGE_NLIST: copy(M->nlist.p, (size_t)nloc * m.nnei * 4); break;
      case DP_STAGE_EXT_COORD: copy(M->ext.p, (size_t)nall * 24); break;
      case DP_STAGE_EXT_TYPE: copy(M->ext_type.p, (size_t)nall * 4); break;
      case DP_STAGE_MAPPING:
        if (!M->last_standalone) throw ApiError{DP_ERR_ARG, "no mapping on the LAMMPS path"};
        copy(M->mapping.p, (size_t)nall * 4);
        break;
      case DP_STAGE_DESCRPT:
        if (M->kind == dp_model::kDpa4c)
          throw ApiError{DP_ERR_ARG, "the DPA4C path keeps its descriptor in registers"};
        if (M->host.axis == 16 && M->nbucket > 0) {
          // not stored by the evaluation: form D from the saved Tsec
          void* Dp = need<char>(M, M->D, (size_t)M->nbucket * Dn * net_esize);
          launch_descriptor(nullptr, desc_args(M, M->Tt.p, Dp), net_esize == 4);
        }
        copy_bucket(M->D.p, Dn, net_esize);
        break;
      case DP_STAGE_DEDD:
        if (M->kind == dp_model::kDpa4c)
          throw ApiError{DP_ERR_ARG, "the DPA4C path keeps dE/dD in registers"};
        if (!M->dd_valid)
          throw ApiError{DP_ERR_ARG,
                         "dE/dD was not stored: call dp_debug_keep(handle, 1) before the "
                         "evaluation"};
        copy_bucket(M->dD.p, Dn, net_esize);
        break;
      case DP_STAGE_ATOM_ENERGY:
        if (M->kind == dp_model::kDpa4c) copy(M->e_bucket.p, (size_t)nloc * 8);
        else copy_bucket(M->e_bucket.p, 1, 8);
        break;
      case DP_STAGE_C4_MOMENTS: copy(M->c4_mom.p, (size_t)nloc * kC4Mom * 4); break;
      case DP_STAGE_C4_COTANGENTS: copy(M->c4_cot.p, (size_t)nloc * kC4Mom * 4); break;
      case DP_STAGE_EDGE_GRAD:
        if (!M->eg_valid)
          throw ApiError{DP_ERR_ARG,
                         "edge gradients were not stored: call dp_debug_keep(handle, 1) before "
                         "the evaluation"};
        copy(M->edge_grad.p, (size_t)nloc * m.nnei * 24);
        break;
      default: throw ApiError{DP_ERR_ARG, "unknown stage"};
    }
  });
  return rc == DP_OK ? result : rc;
}

int dp_stage_times(dp_model* M, int enable, double* times, int n, char* names, size_t names_len) {
  if (!M) return DP_ERR_ARG;
  if (M->timing != (enable != 0)) {
    // start (or stop) timing afresh: sets recorded before are not read
    M->ev_pending = 0;
    M->st_count = 0;
    for (double& v : M->st_sum) v = 0.0;
  }
  M->timing = enable != 0;
  for (int q = 0; q < std::min(n, (int)kNumStages); ++q) times[q] = M->stage_ms[q];
  if (names && names_len) {
    std::string all;
    for (int q = 0; q < kNumStages; ++q) {
      all += kStageNames[q];
      all.push_back('\0');
    }
    std::memcpy(names, all.data(), std::min(names_len, all.size()));
  }
  return kNumStages;
}

size_t dp_device_bytes(const dp_model* M) { return M ? M->bytes_peak : 0; }

int dp_debug_keep(dp_model* M, int keep) {
  if (!M) return DP_ERR_ARG;
  M->keep_edge_grad = keep != 0;
  return DP_OK;
}

int dp_debug_fused_rows(dp_model* M, int rows) {
  if (!M || rows < 0) return DP_ERR_ARG;
  M->fused_ddt_rows = rows;
  return DP_OK;
}

}  // extern "C"
