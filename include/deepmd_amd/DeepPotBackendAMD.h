// deepmd_amd/DeepPotBackendAMD.h — this library as a backend under the
// reference's own deepmd::DeepPot, beside DeepPotPTExpt
// (deepmd-op/overlays/api_cc/include/DeepPotPTExpt.h:37): a header-only class
// template that implements every pure virtual of the reference's
// deepmd::DeepPotBackend (deepmd-op/overlays/api_cc/include/DeepPot.h:23-155
// and the device entries :395-445) over the C ABI of dp_amd.h.
//
// The template takes the reference's own types, so this header needs none of
// upstream's headers and defines nothing in namespace deepmd:
//   Base       deepmd::DeepPotBackend
//   Nlist      deepmd::InputNlist   (fields inum, ilist, numneigh, firstneigh)
//   Exception  deepmd::deepmd_exception (constructible from std::string)
// A maintainer adds, inside upstream's api_cc,
//   class DeepPotAMD final
//       : public deepmd_amd::DeepPotBackendAMD<DeepPotBackend, InputNlist,
//                                              deepmd_exception> {
//     using DeepPotBackendAMD::DeepPotBackendAMD;
//   };
// and lets DeepPot::init choose it for this library's model files, as it
// chooses DeepPotPTExpt for ".pt2": before the choice by file extension,
//   std::string head = file_content.substr(0, 8);  // else the file's first 8 bytes
//   if (head == "DPAMDSEA" || head == "DPAMDC4N") {
//     dp = std::make_shared<deepmd::DeepPotAMD>(model, gpu_rank, file_content);
//     inited = true;
//     return;
//   }
// The pair style and the rest of the reference stay unchanged.
//
// Conventions are the reference's: coord [nframes][natoms][3], box
// [nframes][9] (LAMMPS-shaped, lower-triangular) or empty (open system),
// ener one value per frame, force / atom_virial over all atoms (ghost
// contributions left in ghost slots with a neighbour list), virial [9]
// per frame, atomic outputs only when `atomic`. The evaluation precision is
// the model file's (DP_PREC_MODEL). fparam, aparam and charge_spin are not
// used by these model families and must be empty.
#pragma once

#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../dp_amd.h"

namespace deepmd_amd {

namespace detail {
// The list's neighbour mask (LAMMPS' NEIGHMASK, set by InputNlist::set_mask)
// when the list type carries one, else none.
template <class T, class = void>
struct has_mask : std::false_type {};
template <class T>
struct has_mask<T, std::void_t<decltype(std::declval<const T&>().mask)>> : std::true_type {};
template <class T>
int mask_of(const T& nl) {
  if constexpr (has_mask<T>::value) return (int)nl.mask;
  else return 0;
}
}  // namespace detail

template <class Base, class Nlist, class Exception>
class DeepPotBackendAMD : public Base {
 public:
  DeepPotBackendAMD() = default;
  DeepPotBackendAMD(const std::string& model, const int& gpu_rank = 0,
                    const std::string& file_content = "") {
    init(model, gpu_rank, file_content);
  }
  ~DeepPotBackendAMD() override {
    if (h_) dp_destroy(h_);
  }
  DeepPotBackendAMD(const DeepPotBackendAMD&) = delete;
  DeepPotBackendAMD& operator=(const DeepPotBackendAMD&) = delete;

  void init(const std::string& model, const int& gpu_rank = 0,
            const std::string& file_content = "") override {
    if (h_) {
      dp_destroy(h_);
      h_ = nullptr;
    }
    dp_model* h = nullptr;
    const int rc = dp_create(model.c_str(), gpu_rank,
                             file_content.empty() ? nullptr : file_content.data(),
                             file_content.size(), DP_PREC_MODEL, &h);
    if (rc != DP_OK) {
      const std::string msg = h ? dp_last_error(h) : "dp_create failed";
      if (h) dp_destroy(h);
      throw Exception("DeePMD-kit (MI355X backend) init: " + msg);
    }
    h_ = h;
    check(dp_get_info(h_, &info_));
  }

  // ---- metadata (DeepPotPTExpt.h:103-154 of the reference) ----------------
  double cutoff() const { return info_.rcut; }
  int numb_types() const { return info_.ntypes; }
  int numb_types_spin() const { return 0; }
  int dim_fparam() const { return info_.dim_fparam; }
  int dim_aparam() const { return info_.dim_aparam; }
  bool is_aparam_nall() const { return false; }
  bool has_default_fparam() const { return false; }
  void get_type_map(std::string& type_map) {
    type_map.clear();
    for (int t = 0; t < info_.ntypes; ++t) {
      if (t) type_map += ' ';
      type_map += info_.type_map[t];
    }
  }

  // ---- host entry points ---------------------------------------------------
  // (the base's charge_spin forms, which forward to these, stay visible)
  using Base::computew;
  using Base::computew_mixed_type;
  void computew(std::vector<double>& ener, std::vector<double>& force,
                std::vector<double>& virial, std::vector<double>& atom_energy,
                std::vector<double>& atom_virial, const std::vector<double>& coord,
                const std::vector<int>& atype, const std::vector<double>& box,
                const std::vector<double>& fparam, const std::vector<double>& aparam,
                const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, false, 1, box, nullptr,
           0, 0, fparam.size() + aparam.size(), atomic);
  }
  void computew(std::vector<double>& ener, std::vector<float>& force, std::vector<float>& virial,
                std::vector<float>& atom_energy, std::vector<float>& atom_virial,
                const std::vector<float>& coord, const std::vector<int>& atype,
                const std::vector<float>& box, const std::vector<float>& fparam,
                const std::vector<float>& aparam, const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, false, 1, box, nullptr,
           0, 0, fparam.size() + aparam.size(), atomic);
  }
  void computew(std::vector<double>& ener, std::vector<double>& force,
                std::vector<double>& virial, std::vector<double>& atom_energy,
                std::vector<double>& atom_virial, const std::vector<double>& coord,
                const std::vector<int>& atype, const std::vector<double>& box, const int nghost,
                const Nlist& inlist, const int& ago, const std::vector<double>& fparam,
                const std::vector<double>& aparam, const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, false, 1, box, &inlist,
           nghost, ago, fparam.size() + aparam.size(), atomic);
  }
  void computew(std::vector<double>& ener, std::vector<float>& force, std::vector<float>& virial,
                std::vector<float>& atom_energy, std::vector<float>& atom_virial,
                const std::vector<float>& coord, const std::vector<int>& atype,
                const std::vector<float>& box, const int nghost, const Nlist& inlist,
                const int& ago, const std::vector<float>& fparam,
                const std::vector<float>& aparam, const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, false, 1, box, &inlist,
           nghost, ago, fparam.size() + aparam.size(), atomic);
  }
  void computew_mixed_type(std::vector<double>& ener, std::vector<double>& force,
                           std::vector<double>& virial, std::vector<double>& atom_energy,
                           std::vector<double>& atom_virial, const int& nframes,
                           const std::vector<double>& coord, const std::vector<int>& atype,
                           const std::vector<double>& box, const std::vector<double>& fparam,
                           const std::vector<double>& aparam, const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, true, nframes, box,
           nullptr, 0, 0, fparam.size() + aparam.size(), atomic);
  }
  void computew_mixed_type(std::vector<double>& ener, std::vector<float>& force,
                           std::vector<float>& virial, std::vector<float>& atom_energy,
                           std::vector<float>& atom_virial, const int& nframes,
                           const std::vector<float>& coord, const std::vector<int>& atype,
                           const std::vector<float>& box, const std::vector<float>& fparam,
                           const std::vector<float>& aparam, const bool atomic) override {
    frames(ener, force, virial, atom_energy, atom_virial, coord, atype, true, nframes, box,
           nullptr, 0, 0, fparam.size() + aparam.size(), atomic);
  }

  // ---- device entry points (DeepPot.h:395-445 of the reference) ------------
  bool supports_device_edge_inference() const override { return true; }
  bool uses_fp32_edge_vectors() const override { return false; }
  bool uses_canonical_graph_inference() const override {
    return info_.model_kind == DP_MODEL_DPA4C;
  }
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const double* d_edge_vec, const int nloc, const int nedge) override {
    check(dp_compute_edges_device(h_, d_atom_energy, d_force, d_atom_virial, d_coord, d_atype,
                                  d_edge_index, d_edge_vec, nloc, nedge, nloc, nullptr));
  }
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const double* d_edge_vec, const int nloc, const int nedge,
                         const std::vector<double>& fparam, const std::vector<double>& aparam,
                         const int nall_nodes, const Nlist* comm_nlist) override {
    no_params(fparam.size() + aparam.size());
    (void)comm_nlist;  // single rank: the halo is the caller's
    check(dp_compute_edges_device(h_, d_atom_energy, d_force, d_atom_virial, d_coord, d_atype,
                                  d_edge_index, d_edge_vec, nloc, nedge, nall_nodes, nullptr));
  }
  void compute_edges_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                         const double* d_coord, const int* d_atype, const int* d_edge_index,
                         const float* d_edge_vec, const int nloc, const int nedge,
                         const std::vector<double>& fparam, const std::vector<double>& aparam,
                         const int nall_nodes, const Nlist* comm_nlist) override {
    no_params(fparam.size() + aparam.size());
    (void)comm_nlist;
    check(dp_compute_edges_device_f32(h_, d_atom_energy, d_force, d_atom_virial, d_coord,
                                      d_atype, d_edge_index, d_edge_vec, nloc, nedge, nall_nodes,
                                      nullptr));
  }
  void compute_canonical_graph_gpu(double* d_atom_energy, double* d_force, double* d_atom_virial,
                                   const std::int64_t* d_atype, const std::uint32_t* d_source,
                                   const float* d_edge_vec,
                                   const std::int64_t* d_destination_row_ptr,
                                   const std::int64_t* d_source_row_ptr,
                                   const std::uint32_t* d_source_order, const int nloc,
                                   const int nall_nodes, const std::int64_t edge_storage) override {
    check(dp_compute_canonical_graph_device(h_, d_atom_energy, d_force, d_atom_virial, d_atype,
                                            d_source, d_edge_vec, d_destination_row_ptr,
                                            d_source_row_ptr, d_source_order, nloc, nall_nodes,
                                            edge_storage, nullptr));
  }

  dp_model* handle() const { return h_; }

 private:
  dp_model* h_ = nullptr;
  dp_model_info info_{};

  void check(int rc) const {
    if (rc != DP_OK)
      throw Exception(std::string("DeePMD-kit (MI355X backend): ") +
                      (h_ ? dp_last_error(h_) : "no model loaded"));
  }
  void require_init() const {
    if (!h_) throw Exception("DeePMD-kit (MI355X backend): init() was not called");
  }
  static void no_params(size_t n) {
    if (n) throw Exception("se_e2_a and DPA4C-Nano models take no fparam / aparam");
  }

  // Frames one after another; with typed frames atype holds nframes x natoms
  // types (computew_mixed_type), otherwise the types are shared and the frame
  // count follows from coord. A neighbour list serves every frame (the first
  // with the caller's ago, the rest re-filtered as cached).
  template <typename V>
  void frames(std::vector<double>& ener, std::vector<V>& force, std::vector<V>& virial,
              std::vector<V>& atom_energy, std::vector<V>& atom_virial,
              const std::vector<V>& coord, const std::vector<int>& atype, bool typed_frames,
              int nframes_given, const std::vector<V>& box, const Nlist* nl, int nghost, int ago,
              size_t nparams, bool atomic) {
    require_init();
    no_params(nparams);
    size_t nframes = 1, natoms = atype.size();
    if (typed_frames) {
      if (nframes_given <= 0 || atype.size() % (size_t)nframes_given)
        throw Exception("atype size must be nframes * natoms");
      nframes = (size_t)nframes_given;
      natoms = atype.size() / nframes;
    } else if (natoms > 0) {
      if (coord.size() % (3 * natoms)) throw Exception("coord size must be nframes * natoms * 3");
      nframes = coord.size() / (3 * natoms);
    } else if (!box.empty()) {
      nframes = box.size() / 9;
    }
    if (coord.size() != nframes * natoms * 3)
      throw Exception("coord size must be nframes * natoms * 3");
    if (!box.empty() && box.size() != 9 * nframes) throw Exception("box size must be nframes * 9");
    ener.assign(nframes, 0.0);
    force.assign(nframes * natoms * 3, V(0));
    virial.assign(nframes * 9, V(0));
    atom_energy.assign(atomic ? nframes * natoms : 0, V(0));
    atom_virial.assign(atomic ? nframes * natoms * 9 : 0, V(0));
    const int n = (int)natoms;
    std::vector<double> c(3 * natoms), b(box.empty() ? 0 : 9), f(3 * natoms), v(9),
        ae(atomic ? natoms : 0), av(atomic ? 9 * natoms : 0);
    std::vector<int> t(natoms);
    for (size_t fr = 0; fr < nframes; ++fr) {
      for (size_t q = 0; q < 3 * natoms; ++q) c[q] = (double)coord[fr * 3 * natoms + q];
      for (size_t q = 0; q < b.size(); ++q) b[q] = (double)box[fr * 9 + q];
      for (size_t q = 0; q < natoms; ++q) t[q] = atype[(typed_frames ? fr * natoms : 0) + q];
      const double* bp = b.empty() ? nullptr : b.data();
      if (nl)
        check(dp_compute_nlist(h_, n, nghost, c.data(), t.data(), bp, nl->inum, nl->ilist,
                               nl->numneigh, nl->firstneigh, detail::mask_of(*nl),
                               fr ? 1 : ago, &ener[fr],
                               f.data(), v.data(), atomic ? ae.data() : nullptr,
                               atomic ? av.data() : nullptr));
      else
        check(dp_compute(h_, n, c.data(), t.data(), bp, &ener[fr], f.data(), v.data(),
                         atomic ? ae.data() : nullptr, atomic ? av.data() : nullptr));
      for (size_t q = 0; q < 3 * natoms; ++q) force[fr * 3 * natoms + q] = (V)f[q];
      for (size_t q = 0; q < 9; ++q) virial[fr * 9 + q] = (V)v[q];
      if (atomic) {
        for (size_t q = 0; q < natoms; ++q) atom_energy[fr * natoms + q] = (V)ae[q];
        for (size_t q = 0; q < 9 * natoms; ++q) atom_virial[fr * 9 * natoms + q] = (V)av[q];
      }
    }
  }
};

}  // namespace deepmd_amd
