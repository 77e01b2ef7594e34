// deepmd_amd/DeepPot.h — header-only C++ façade over dp_amd.h that keeps the
// surface `pair_style deepmd` calls on the reference's deepmd::DeepPot
// (deepmd-op/overlays/api_cc/include/DeepPot.h:451-926) and the upstream
// InputNlist type (fields evidenced at lammps-deepmd-plugin/src/pair_deepmd.cpp:355-364).
// Failures throw deepmd::deepmd_exception, which the pair style turns into
// error->one (pair_deepmd.cpp:372-374).
//
// Link with -ldpamd. The interface is double precision; the float overloads
// convert at the boundary, as the reference's compute<float> does. The
// evaluation precision is chosen at init: DP_PREC_FP64 (default) or
// DP_PREC_MIXED (fp32 nets, fp64 env matrix / forces / virial). Upstream the
// precision is a property of the trained model, so init() keeps the
// reference's three arguments and reads the choice from the environment
// variable DPAMD_PRECISION ("fp64" or "mixed") unless it is passed explicitly.
#pragma once

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <cstdint>
#include <string>
#include <vector>

#include "../dp_amd.h"

namespace deepmd {

typedef double ENERGYTYPE;

class deepmd_exception : public std::runtime_error {
 public:
  explicit deepmd_exception(const std::string& msg) : std::runtime_error(msg) {}
};

// LAMMPS neighbour list handed to the model (full list, with skin). The
// communication fields are carried for source compatibility; this build is
// single-rank and does not read them.
struct InputNlist {
  int inum = 0;
  int* ilist = nullptr;
  int* numneigh = nullptr;
  int** firstneigh = nullptr;
  int nswap = 0;
  int* sendnum = nullptr;
  int* recvnum = nullptr;
  int* firstrecv = nullptr;
  int** sendlist = nullptr;
  int* sendproc = nullptr;
  int* recvproc = nullptr;
  void* world = nullptr;
  int nprocs = 1;
  int mask = 0;
  int* mapping = nullptr;
  InputNlist() = default;
  InputNlist(int inum_, int* ilist_, int* numneigh_, int** firstneigh_)
      : inum(inum_), ilist(ilist_), numneigh(numneigh_), firstneigh(firstneigh_) {}
  InputNlist(int inum_, int* ilist_, int* numneigh_, int** firstneigh_, int nswap_,
             int* sendnum_, int* recvnum_, int* firstrecv_, int** sendlist_, int* sendproc_,
             int* recvproc_, void* world_, int nprocs_ = 1)
      : inum(inum_), ilist(ilist_), numneigh(numneigh_), firstneigh(firstneigh_),
        nswap(nswap_), sendnum(sendnum_), recvnum(recvnum_), firstrecv(firstrecv_),
        sendlist(sendlist_), sendproc(sendproc_), recvproc(recvproc_), world(world_),
        nprocs(nprocs_) {}
  void set_mask(int m) { mask = m; }
  void set_mapping(int* m) { mapping = m; }
};

class DeepPot {
 public:
  DeepPot() = default;
  DeepPot(const std::string& model, const int& gpu_rank = 0,
          const std::string& file_content = "") {
    init(model, gpu_rank, file_content);
  }
  ~DeepPot() {
    if (h_) dp_destroy(h_);
  }
  DeepPot(const DeepPot&) = delete;
  DeepPot& operator=(const DeepPot&) = delete;

  void init(const std::string& model, const int& gpu_rank = 0,
            const std::string& file_content = "", int precision = -1) {
    if (h_) {
      dp_destroy(h_);
      h_ = nullptr;
    }
    if (precision < 0) {
      const char* env = std::getenv("DPAMD_PRECISION");
      precision = DP_PREC_FP64;
      if (env && std::strcmp(env, "mixed") == 0) precision = DP_PREC_MIXED;
      else if (env && *env && std::strcmp(env, "fp64") != 0)
        throw deepmd_exception(std::string("DPAMD_PRECISION must be fp64 or mixed, got ") + env);
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

  double cutoff() const { return info_.rcut; }
  int numb_types() const { return info_.ntypes; }
  int numb_types_spin() const { return 0; }
  int dim_fparam() const { return info_.dim_fparam; }
  int dim_aparam() const { return info_.dim_aparam; }
  int dim_chg_spin() const { return 0; }
  void get_type_map(std::string& type_map) const {
    type_map.clear();
    for (int t = 0; t < info_.ntypes; ++t) {
      if (t) type_map += " ";
      type_map += info_.type_map[t];
    }
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

  dp_model* handle() const { return h_; }

 private:
  dp_model* h_ = nullptr;
  dp_model_info info_{};

  void check(int rc) const {
    if (rc != DP_OK) throw deepmd_exception(std::string("DeePMD-kit (MI355X): ") + dp_last_error(h_));
  }
  void require_init() const {
    if (!h_) throw deepmd_exception("DeePMD-kit (MI355X): model not initialised");
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

}  // namespace deepmd
