// deepmd_amd/DeepPot.h — header-only C++ façade over dp_amd.h that keeps the
// surface `pair_style deepmd` calls on the reference's deepmd::DeepPot and
// deepmd::DeepPotModelDevi (deepmd-op/overlays/api_cc/include/DeepPot.h:451-926,
// :928-1104), on top of the model-base types of DeepBaseModel.h. pair_deepmd.h
// of the reference plugin (lammps-deepmd-plugin/src/pair_deepmd.h:16-28,
// :55-56) includes this header under that name and declares a
// deepmd_compat::DeepPot and a deepmd_compat::DeepPotModelDevi.
//
// Link with -ldpamd. The interface is double precision; the float overloads
// convert at the boundary, as the reference's compute<float> does. The
// evaluation precision is a property of the model, as upstream: init() keeps
// the reference's three arguments and evaluates in the precision the model
// file records (DP_PREC_FP64, or DP_PREC_MIXED: fp32 nets, fp64 env matrix /
// forces / virial); a fourth argument overrides it.
//
// Frames: the std::vector<ENERGYTYPE> overloads take nframes configurations
// back to back (coord nframes x natoms x 3, box nframes x 9 or empty) and
// evaluate them one after another; compute_mixed_type also takes per-frame
// types (atype nframes x natoms). With a neighbour list every frame uses the
// caller's list, the first with the caller's `ago`, the others as cached
// (ago = 1: re-filtered on that frame's positions).
#pragma once

#include "DeepBaseModel.h"

namespace deepmd {

class DeepPot : public DeepBaseModel {
 public:
  DeepPot() = default;
  DeepPot(const std::string& model, const int& gpu_rank = 0,
          const std::string& file_content = "") {
    init(model, gpu_rank, file_content);
  }

  void init(const std::string& model, const int& gpu_rank = 0,
            const std::string& file_content = "", int precision = DP_PREC_MODEL) {
    if (h_) {
      dp_destroy(h_);
      h_ = nullptr;
    }
    dp_model* h = nullptr;
    const int rc = dp_create(model.c_str(), gpu_rank,
                             file_content.empty() ? nullptr : file_content.data(),
                             file_content.size(), precision, &h);
    if (rc != DP_OK) {
      const std::string msg = h ? dp_last_error(h) : "dp_create failed";
      if (h) dp_destroy(h);
      throw deepmd_exception("DeePMD-kit (MI355X) init: " + msg);
    }
    h_ = h;
    dp_get_info(h_, &info_);
  }

  // Neither model family has a charge / spin input (dim_chg_spin() == 0):
  // only the empty condition is accepted.
  void set_charge_spin(const std::vector<double>& charge_spin) {
    if (!charge_spin.empty())
      throw deepmd_exception("DeePMD-kit (MI355X): the model has no charge/spin input");
  }

  // compute(ener, force, virial, coord, atype, box[, fparam, aparam, charge_spin])
  template <typename VALUETYPE>
  void compute(ENERGYTYPE& ener, std::vector<VALUETYPE>& force, std::vector<VALUETYPE>& virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<VALUETYPE> ae, av;
    compute_impl(ener, force, virial, ae, av, false, coord, atype, box, fparam, aparam,
                 charge_spin);
  }
  // compute(ener, force, virial, atom_energy, atom_virial, coord, atype, box[, ...])
  template <typename VALUETYPE>
  void compute(ENERGYTYPE& ener, std::vector<VALUETYPE>& force, std::vector<VALUETYPE>& virial,
               std::vector<VALUETYPE>& atom_energy, std::vector<VALUETYPE>& atom_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    compute_impl(ener, force, virial, atom_energy, atom_virial, true, coord, atype, box, fparam,
                 aparam, charge_spin);
  }
  // compute(ener, force, virial, coord, atype, box, nghost, lmp_list, ago[, ...])
  template <typename VALUETYPE>
  void compute(ENERGYTYPE& ener, std::vector<VALUETYPE>& force, std::vector<VALUETYPE>& virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box, const int nghost, const InputNlist& lmp_list,
               const int& ago, const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<VALUETYPE> ae, av;
    compute_nlist_impl(ener, force, virial, ae, av, false, coord, atype, box, nghost, lmp_list,
                       ago, fparam, aparam, charge_spin);
  }
  // compute(ener, force, virial, atom_energy, atom_virial, coord, atype, box, nghost, lmp_list, ago[, ...])
  template <typename VALUETYPE>
  void compute(ENERGYTYPE& ener, std::vector<VALUETYPE>& force, std::vector<VALUETYPE>& virial,
               std::vector<VALUETYPE>& atom_energy, std::vector<VALUETYPE>& atom_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box, const int nghost, const InputNlist& lmp_list,
               const int& ago, const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    compute_nlist_impl(ener, force, virial, atom_energy, atom_virial, true, coord, atype, box,
                       nghost, lmp_list, ago, fparam, aparam, charge_spin);
  }

  // Frames back to back: ener[nframes], force nframes x natoms x 3, virial
  // nframes x 9 (DeepPot.h:492-502, :539-549, :577-587, :631-644 of the
  // reference api_cc/include).
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
               std::vector<VALUETYPE>& virial, const std::vector<VALUETYPE>& coord,
               const std::vector<int>& atype, const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<VALUETYPE> ae, av;
    frames_impl(ener, force, virial, ae, av, false, coord, atype, false, box, nullptr, 0, 0,
                fparam, aparam, charge_spin);
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
               std::vector<VALUETYPE>& virial, std::vector<VALUETYPE>& atom_energy,
               std::vector<VALUETYPE>& atom_virial, const std::vector<VALUETYPE>& coord,
               const std::vector<int>& atype, const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    frames_impl(ener, force, virial, atom_energy, atom_virial, true, coord, atype, false, box,
                nullptr, 0, 0, fparam, aparam, charge_spin);
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
               std::vector<VALUETYPE>& virial, const std::vector<VALUETYPE>& coord,
               const std::vector<int>& atype, const std::vector<VALUETYPE>& box,
               const int nghost, const InputNlist& lmp_list, const int& ago,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<VALUETYPE> ae, av;
    frames_impl(ener, force, virial, ae, av, false, coord, atype, false, box, &lmp_list, nghost,
                ago, fparam, aparam, charge_spin);
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
               std::vector<VALUETYPE>& virial, std::vector<VALUETYPE>& atom_energy,
               std::vector<VALUETYPE>& atom_virial, const std::vector<VALUETYPE>& coord,
               const std::vector<int>& atype, const std::vector<VALUETYPE>& box,
               const int nghost, const InputNlist& lmp_list, const int& ago,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    frames_impl(ener, force, virial, atom_energy, atom_virial, true, coord, atype, false, box,
                &lmp_list, nghost, ago, fparam, aparam, charge_spin);
  }
  // Per-frame types (atype nframes x natoms), DeepPot.h:700-760 of the
  // reference api_cc/include; the scalar-energy forms take one frame.
  template <typename VALUETYPE>
  void compute_mixed_type(ENERGYTYPE& ener, std::vector<VALUETYPE>& force,
                          std::vector<VALUETYPE>& virial, const int& nframes,
                          const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
                          const std::vector<VALUETYPE>& box,
                          const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
                          const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
                          const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<ENERGYTYPE> e;
    std::vector<VALUETYPE> ae, av;
    one_frame(nframes);
    frames_impl(e, force, virial, ae, av, false, coord, atype, true, box, nullptr, 0, 0, fparam,
                aparam, charge_spin);
    ener = e[0];
  }
  template <typename VALUETYPE>
  void compute_mixed_type(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
                          std::vector<VALUETYPE>& virial, const int& nframes,
                          const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
                          const std::vector<VALUETYPE>& box,
                          const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
                          const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
                          const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<VALUETYPE> ae, av;
    frames_impl(ener, force, virial, ae, av, false, coord, atype, true, box, nullptr, 0, 0,
                fparam, aparam, charge_spin, nframes);
  }
  template <typename VALUETYPE>
  void compute_mixed_type(ENERGYTYPE& ener, std::vector<VALUETYPE>& force,
                          std::vector<VALUETYPE>& virial, std::vector<VALUETYPE>& atom_energy,
                          std::vector<VALUETYPE>& atom_virial, const int& nframes,
                          const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
                          const std::vector<VALUETYPE>& box,
                          const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
                          const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
                          const std::vector<double>& charge_spin = std::vector<double>()) {
    std::vector<ENERGYTYPE> e;
    one_frame(nframes);
    frames_impl(e, force, virial, atom_energy, atom_virial, true, coord, atype, true, box,
                nullptr, 0, 0, fparam, aparam, charge_spin);
    ener = e[0];
  }
  template <typename VALUETYPE>
  void compute_mixed_type(std::vector<ENERGYTYPE>& ener, std::vector<VALUETYPE>& force,
                          std::vector<VALUETYPE>& virial, std::vector<VALUETYPE>& atom_energy,
                          std::vector<VALUETYPE>& atom_virial, const int& nframes,
                          const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
                          const std::vector<VALUETYPE>& box,
                          const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
                          const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
                          const std::vector<double>& charge_spin = std::vector<double>()) {
    frames_impl(ener, force, virial, atom_energy, atom_virial, true, coord, atype, true, box,
                nullptr, 0, 0, fparam, aparam, charge_spin, nframes);
  }

  // Device-resident step on device pointers (dp_compute_device, or with
  // async = true dp_compute_device_async: queued on `stream` with no host
  // synchronisation; sync() waits and reports a deferred capacity error). The
  // step the reference hands between the MD engine's and the model's streams
  // (DeepPot.h:14-18 and :395-445 of deepmd-op/overlays/api_cc/include).
  void compute_device(double* d_energy, double* d_force, double* d_virial, double* d_atom_energy,
                      double* d_atom_virial, const double* d_coord, const int* d_atype,
                      const int natoms, const std::vector<double>& box, const int ago = 1,
                      void* stream = nullptr, const bool async = false) {
    require_init();
    if (box.size() != 9) throw deepmd_exception("DeePMD-kit (MI355X): box must hold 9 values");
    check((async ? dp_compute_device_async : dp_compute_device)(
        h_, natoms, d_coord, d_atype, box.data(), ago, d_energy, d_force, d_virial, d_atom_energy,
        d_atom_virial, stream));
  }
  void sync() {
    require_init();
    check(dp_sync(h_));
  }

  // DPA4C models: the compact canonical graph entry, same signature and
  // argument meaning as DeepPot::compute_canonical_graph_gpu
  // (deepmd-op/overlays/api_cc/include/DeepPot.h:430-442); dp_compute_canonical_graph_device.
  void compute_canonical_graph_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                                   const std::int64_t* d_atype, const std::uint32_t* d_source,
                                   const float* d_edge_vec,
                                   const std::int64_t* d_destination_row_ptr,
                                   const std::int64_t* d_source_row_ptr,
                                   const std::uint32_t* d_source_order, const int nloc,
                                   const int nall_nodes, const std::int64_t edge_storage,
                                   void* stream = nullptr) {
    require_init();
    check(dp_compute_canonical_graph_device(h_, d_atom_energy, d_force, d_atom_virial, d_atype,
                                            d_source, d_edge_vec, d_destination_row_ptr,
                                            d_source_row_ptr, d_source_order, nloc, nall_nodes,
                                            edge_storage, stream));
  }
  // Device edge-graph entry, same overloads and argument meaning as
  // DeepPot::compute_edges_gpu (deepmd-op/overlays/api_cc/include/DeepPot.h:395-429):
  // edge_index [2][nedge] holds the source node in row 0 and the destination
  // centre (< nloc) in row 1, edge_vec = r_source - r_centre. Both model kinds
  // take no fparam / aparam and exchange no node features between ranks, so
  // comm_nlist is not read. dp_compute_edges_device / _f32.
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const double* d_edge_vec, const int nloc, const int nedge) {
    edges_impl(d_atom_energy, d_force, d_atom_virial, d_coord, d_atype, d_edge_index, d_edge_vec,
               nloc, nedge, nloc);
  }
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const double* d_edge_vec, const int nloc, const int nedge,
                         const std::vector<double>& fparam, const std::vector<double>& aparam,
                         const int nall_nodes, const InputNlist* comm_nlist) {
    (void)comm_nlist;
    no_params(fparam, aparam, std::vector<double>());
    edges_impl(d_atom_energy, d_force, d_atom_virial, d_coord, d_atype, d_edge_index, d_edge_vec,
               nloc, nedge, nall_nodes);
  }
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const float* d_edge_vec, const int nloc, const int nedge,
                         const std::vector<double>& fparam, const std::vector<double>& aparam,
                         const int nall_nodes, const InputNlist* comm_nlist) {
    (void)comm_nlist;
    no_params(fparam, aparam, std::vector<double>());
    edges_impl(d_atom_energy, d_force, d_atom_virial, d_coord, d_atype, d_edge_index, d_edge_vec,
               nloc, nedge, nall_nodes);
  }
  bool uses_canonical_graph_inference() const { return info_.model_kind == DP_MODEL_DPA4C; }
  bool uses_fp32_edge_vectors() const { return info_.model_kind == DP_MODEL_DPA4C; }
  bool supports_device_edge_inference() const { return true; }

 private:
  static void one_frame(int nframes) {
    if (nframes != 1)
      throw deepmd_exception("DeePMD-kit (MI355X): a scalar energy holds one frame, got " +
                             std::to_string(nframes));
  }
  // nframes_given > 0 (mixed-type form): atype holds nframes x natoms types;
  // otherwise the types are shared and nframes follows from coord.
  template <typename V>
  void frames_impl(std::vector<ENERGYTYPE>& ener, std::vector<V>& force, std::vector<V>& virial,
                   std::vector<V>& atom_energy, std::vector<V>& atom_virial, bool atomic,
                   const std::vector<V>& coord, const std::vector<int>& atype, bool typed_frames,
                   const std::vector<V>& box, const InputNlist* nl, int nghost, int ago,
                   const std::vector<V>& fparam, const std::vector<V>& aparam,
                   const std::vector<double>& cs, int nframes_given = 1) {
    require_init();
    size_t nframes = 1, natoms = atype.size();
    if (typed_frames) {
      if (nframes_given <= 0 || atype.size() % (size_t)nframes_given)
        throw deepmd_exception("atype size must be nframes * natoms");
      nframes = (size_t)nframes_given;
      natoms = atype.size() / nframes;
    } else if (natoms > 0) {
      if (coord.size() % (3 * natoms)) throw deepmd_exception("coord size must be nframes * natoms * 3");
      nframes = coord.size() / (3 * natoms);
    } else if (!box.empty()) {
      nframes = box.size() / 9;
    }
    if (coord.size() != nframes * natoms * 3)
      throw deepmd_exception("coord size must be nframes * natoms * 3");
    if (!box.empty() && box.size() != 9 * nframes)
      throw deepmd_exception("box size must be nframes * 9");
    ener.assign(nframes, 0.0);
    force.clear();
    virial.clear();
    atom_energy.clear();
    atom_virial.clear();
    for (size_t f = 0; f < nframes; ++f) {
      const std::vector<V> c(coord.begin() + f * natoms * 3, coord.begin() + (f + 1) * natoms * 3);
      const std::vector<int> t = typed_frames
          ? std::vector<int>(atype.begin() + f * natoms, atype.begin() + (f + 1) * natoms)
          : atype;
      const std::vector<V> b = box.empty() ? std::vector<V>()
                                           : std::vector<V>(box.begin() + f * 9, box.begin() + (f + 1) * 9);
      std::vector<V> ff, vv, ae, av;
      if (nl)
        compute_nlist_impl(ener[f], ff, vv, ae, av, atomic, c, t, b, nghost, *nl, f ? 1 : ago,
                           fparam, aparam, cs);
      else
        compute_impl(ener[f], ff, vv, ae, av, atomic, c, t, b, fparam, aparam, cs);
      force.insert(force.end(), ff.begin(), ff.end());
      virial.insert(virial.end(), vv.begin(), vv.end());
      if (atomic) {
        atom_energy.insert(atom_energy.end(), ae.begin(), ae.end());
        atom_virial.insert(atom_virial.end(), av.begin(), av.end());
      }
    }
  }
  template <typename V>
  static void no_params(const std::vector<V>& fparam, const std::vector<V>& aparam,
                        const std::vector<double>& cs) {
    if (!fparam.empty() || !aparam.empty() || !cs.empty())
      throw deepmd_exception("se_e2_a and DPA4C-Nano models take no fparam / aparam / charge_spin");
  }
  void edges_impl(double* ae, double* f, double* av, const double* coord, const int* atype,
                  const int* ei, const double* vec, int nloc, int nedge, int nall_nodes) {
    require_init();
    check(dp_compute_edges_device(h_, ae, f, av, coord, atype, ei, vec, nloc, nedge, nall_nodes,
                                  nullptr));
  }
  void edges_impl(double* ae, double* f, double* av, const double* coord, const int* atype,
                  const int* ei, const float* vec, int nloc, int nedge, int nall_nodes) {
    require_init();
    check(dp_compute_edges_device_f32(h_, ae, f, av, coord, atype, ei, vec, nloc, nedge,
                                      nall_nodes, nullptr));
  }
  template <typename V>
  static std::vector<double> to_double(const std::vector<V>& v) {
    return std::vector<double>(v.begin(), v.end());
  }
  template <typename V>
  static void from_double(std::vector<V>& out, const std::vector<double>& v) {
    out.assign(v.begin(), v.end());
  }

  template <typename V>
  void compute_impl(ENERGYTYPE& ener, std::vector<V>& force, std::vector<V>& virial,
                    std::vector<V>& atom_energy, std::vector<V>& atom_virial, bool atomic,
                    const std::vector<V>& coord, const std::vector<int>& atype,
                    const std::vector<V>& box, const std::vector<V>& fparam,
                    const std::vector<V>& aparam, const std::vector<double>& cs) {
    require_init();
    no_params(fparam, aparam, cs);
    const int n = (int)atype.size();
    if ((int)coord.size() != 3 * n) throw deepmd_exception("coord size must be 3 * natoms");
    if (!box.empty() && box.size() != 9) throw deepmd_exception("box must have 9 entries");
    const std::vector<double> c = to_double(coord), b = to_double(box);
    std::vector<double> f(3 * (size_t)n), v(9), ae, av;
    if (atomic) {
      ae.resize(n);
      av.resize(9 * (size_t)n);
    }
    check(dp_compute(h_, n, c.data(), atype.data(), b.empty() ? nullptr : b.data(), &ener,
                     f.data(), v.data(), atomic ? ae.data() : nullptr,
                     atomic ? av.data() : nullptr));
    from_double(force, f);
    from_double(virial, v);
    if (atomic) {
      from_double(atom_energy, ae);
      from_double(atom_virial, av);
    }
  }

  template <typename V>
  void compute_nlist_impl(ENERGYTYPE& ener, std::vector<V>& force, std::vector<V>& virial,
                          std::vector<V>& atom_energy, std::vector<V>& atom_virial, bool atomic,
                          const std::vector<V>& coord, const std::vector<int>& atype,
                          const std::vector<V>& box, int nghost, const InputNlist& nl, int ago,
                          const std::vector<V>& fparam, const std::vector<V>& aparam,
                          const std::vector<double>& cs) {
    require_init();
    no_params(fparam, aparam, cs);
    const int nall = (int)atype.size();
    if ((int)coord.size() != 3 * nall) throw deepmd_exception("coord size must be 3 * nall");
    const std::vector<double> c = to_double(coord), b = to_double(box);
    std::vector<double> f(3 * (size_t)nall), v(9), ae, av;
    if (atomic) {
      ae.resize(nall);
      av.resize(9 * (size_t)nall);
    }
    check(dp_compute_nlist(h_, nall, nghost, c.data(), atype.data(),
                           b.empty() ? nullptr : b.data(), nl.inum, nl.ilist, nl.numneigh,
                           nl.firstneigh, nl.mask, ago, &ener, f.data(), v.data(),
                           atomic ? ae.data() : nullptr, atomic ? av.data() : nullptr));
    from_double(force, f);
    from_double(virial, v);
    if (atomic) {
      from_double(atom_energy, ae);
      from_double(atom_virial, av);
    }
  }
};

// Several models on the same configuration (pair_deepmd.cpp:426-442 calls
// compute with every model's outputs, :493-530 the deviation statistics).
class DeepPotModelDevi : public DeepBaseModelDevi {
 public:
  DeepPotModelDevi() = default;
  DeepPotModelDevi(const std::vector<std::string>& models, const int& gpu_rank = 0,
                   const std::vector<std::string>& file_contents = std::vector<std::string>()) {
    init(models, gpu_rank, file_contents);
  }
  // Every model is loaded onto the same GPU; they must agree on the cutoff
  // and the number of types, as one neighbour list serves them all.
  void init(const std::vector<std::string>& models, const int& gpu_rank = 0,
            const std::vector<std::string>& file_contents = std::vector<std::string>()) {
    if (models.empty()) throw deepmd_exception("DeePMD-kit (MI355X): no models given");
    if (!file_contents.empty() && file_contents.size() != models.size())
      throw deepmd_exception("DeePMD-kit (MI355X): one file content per model expected");
    dps.clear();
    dpbases.clear();
    for (size_t k = 0; k < models.size(); ++k) {
      auto p = std::make_shared<DeepPot>();
      p->init(models[k], gpu_rank, file_contents.empty() ? std::string() : file_contents[k]);
      if (k && (p->cutoff() != dps[0]->cutoff() || p->numb_types() != dps[0]->numb_types()))
        throw deepmd_exception("DeePMD-kit (MI355X): models differ in cutoff or type count");
      dps.push_back(p);
      dpbases.push_back(p);
    }
    numb_models = (unsigned)dps.size();
  }
  int dim_chg_spin() const { return numb_models > 0 ? dps[0]->dim_chg_spin() : 0; }
  void set_charge_spin(const std::vector<double>& charge_spin) {
    for (auto& p : dps) p->set_charge_spin(charge_spin);
  }

  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& all_ener, std::vector<std::vector<VALUETYPE>>& all_force,
               std::vector<std::vector<VALUETYPE>>& all_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    each(all_ener, all_force, all_virial, [&](DeepPot& d, ENERGYTYPE& e, std::vector<VALUETYPE>& f,
                                              std::vector<VALUETYPE>& v, size_t) {
      d.compute(e, f, v, coord, atype, box, fparam, aparam, charge_spin);
    });
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& all_ener, std::vector<std::vector<VALUETYPE>>& all_force,
               std::vector<std::vector<VALUETYPE>>& all_virial,
               std::vector<std::vector<VALUETYPE>>& all_atom_energy,
               std::vector<std::vector<VALUETYPE>>& all_atom_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box,
               const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    all_atom_energy.assign(models(), {});
    all_atom_virial.assign(models(), {});
    each(all_ener, all_force, all_virial, [&](DeepPot& d, ENERGYTYPE& e, std::vector<VALUETYPE>& f,
                                              std::vector<VALUETYPE>& v, size_t k) {
      d.compute(e, f, v, all_atom_energy[k], all_atom_virial[k], coord, atype, box, fparam,
                aparam, charge_spin);
    });
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& all_ener, std::vector<std::vector<VALUETYPE>>& all_force,
               std::vector<std::vector<VALUETYPE>>& all_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box, const int nghost, const InputNlist& lmp_list,
               const int& ago, const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    each(all_ener, all_force, all_virial, [&](DeepPot& d, ENERGYTYPE& e, std::vector<VALUETYPE>& f,
                                              std::vector<VALUETYPE>& v, size_t) {
      d.compute(e, f, v, coord, atype, box, nghost, lmp_list, ago, fparam, aparam, charge_spin);
    });
  }
  template <typename VALUETYPE>
  void compute(std::vector<ENERGYTYPE>& all_ener, std::vector<std::vector<VALUETYPE>>& all_force,
               std::vector<std::vector<VALUETYPE>>& all_virial,
               std::vector<std::vector<VALUETYPE>>& all_atom_energy,
               std::vector<std::vector<VALUETYPE>>& all_atom_virial,
               const std::vector<VALUETYPE>& coord, const std::vector<int>& atype,
               const std::vector<VALUETYPE>& box, const int nghost, const InputNlist& lmp_list,
               const int& ago, const std::vector<VALUETYPE>& fparam = std::vector<VALUETYPE>(),
               const std::vector<VALUETYPE>& aparam = std::vector<VALUETYPE>(),
               const std::vector<double>& charge_spin = std::vector<double>()) {
    all_atom_energy.assign(models(), {});
    all_atom_virial.assign(models(), {});
    each(all_ener, all_force, all_virial, [&](DeepPot& d, ENERGYTYPE& e, std::vector<VALUETYPE>& f,
                                              std::vector<VALUETYPE>& v, size_t k) {
      d.compute(e, f, v, all_atom_energy[k], all_atom_virial[k], coord, atype, box, nghost,
                lmp_list, ago, fparam, aparam, charge_spin);
    });
  }

 protected:
  std::vector<std::shared_ptr<DeepPot>> dps;

 private:
  template <typename V, class Fn>
  void each(std::vector<ENERGYTYPE>& all_ener, std::vector<std::vector<V>>& all_force,
            std::vector<std::vector<V>>& all_virial, Fn&& fn) {
    if (dps.empty()) throw deepmd_exception("DeePMD-kit (MI355X): no models initialised");
    all_ener.assign(dps.size(), 0.0);
    all_force.assign(dps.size(), {});
    all_virial.assign(dps.size(), {});
    for (size_t k = 0; k < dps.size(); ++k) fn(*dps[k], all_ener[k], all_force[k], all_virial[k], k);
  }
};

}  // namespace deepmd
