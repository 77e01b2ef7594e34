// deepmd_amd/DeepBaseModel.h — the model-base layer of the header-only C++
// façade over dp_amd.h: the types `pair_style deepmd` binds to before it
// knows which model family it runs. pair_base.h of the reference plugin
// (lammps-deepmd-plugin/src/pair_base.h:10-16, :33-36, :61-62) includes this
// header under that name and holds a deepmd_compat::DeepBaseModel& and a
// deepmd_compat::DeepBaseModelDevi& with `namespace deepmd_compat = deepmd;`;
// pair_base.cpp:73 calls deepmd_compat::read_file_to_string and :459
// deep_base.print_summary.
//
// DeepBaseModel and DeepBaseModelDevi are upstream DeePMD-kit types (46fdc3e8,
// api_cc/include/DeepBaseModel.h, absent from the reference tree); their
// method names and the model-deviation statistics below follow upstream's
// documented definitions: the deviation of a per-atom quantity is the root
// mean square over models of the distance to the model average,
//   std_i = sqrt( (1/M) sum_k sum_d (x_k[i*s+d] - avg[i*s+d])^2 ),
// with stride s = 3 for forces and 1 for each virial component, and the
// relative form divides it by |avg_i| + eps.
//
// Failures throw deepmd::deepmd_exception, which the pair style turns into
// error->one (pair_deepmd.cpp:372-374).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <iterator>
#include <memory>
#include <stdexcept>
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

// Reads a whole model file into `file_content` (pair_base.cpp:73 hands the
// content to init() so that every rank reads the file once).
inline void read_file_to_string(std::string model, std::string& file_content) {
  std::ifstream f(model, std::ios::binary);
  if (!f) throw deepmd_exception("DeePMD-kit (MI355X): cannot open model file " + model);
  file_content.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

// One loaded model: a libdpamd handle and its metadata.
class DeepBaseModel {
 public:
  DeepBaseModel() = default;
  virtual ~DeepBaseModel() {
    if (h_) dp_destroy(h_);
  }
  DeepBaseModel(const DeepBaseModel&) = delete;
  DeepBaseModel& operator=(const DeepBaseModel&) = delete;

  double cutoff() const { return info_.rcut; }
  int numb_types() const { return info_.ntypes; }
  int numb_types_spin() const { return 0; }
  int dim_fparam() const { return info_.dim_fparam; }
  int dim_aparam() const { return info_.dim_aparam; }
  int dim_chg_spin() const { return 0; }
  bool is_aparam_nall() const { return false; }
  void get_type_map(std::string& type_map) const {
    type_map.clear();
    for (int t = 0; t < info_.ntypes; ++t) {
      if (t) type_map += " ";
      type_map += info_.type_map[t];
    }
  }
  // Model summary, one line per item, each prefixed by `pre` (the pair
  // style passes "  >>> Info of model(s):"-style prefixes).
  void print_summary(const std::string& pre) const {
    std::string tm;
    get_type_map(tm);
    std::cout << pre << "DeePMD-kit MI355X-native backend (libdpamd, gfx950 HIP kernels)\n";
    if (!h_) {
      std::cout << pre << "model not initialised\n";
      return;
    }
    std::cout << pre << "model kind:   "
              << (info_.model_kind == DP_MODEL_DPA4C ? "DPA4C-Nano" : "se_e2_a") << "\n";
    std::cout << pre << "precision:    "
              << (info_.precision == DP_PREC_MIXED ? "mixed (fp32 nets, fp64 env / force / virial)"
                                                   : "fp64")
              << "\n";
    std::cout << pre << "cutoff:       " << info_.rcut << "\n";
    std::cout << pre << "type map:     " << tm << "\n";
    std::cout << pre << "sel:         ";
    for (int t = 0; t < info_.ntypes; ++t) std::cout << " " << info_.sel[t];
    std::cout << "\n";
  }

  dp_model* handle() const { return h_; }

 protected:
  dp_model* h_ = nullptr;
  dp_model_info info_{};

  void check(int rc) const {
    if (rc != DP_OK) throw deepmd_exception(std::string("DeePMD-kit (MI355X): ") + dp_last_error(h_));
  }
  void require_init() const {
    if (!h_) throw deepmd_exception("DeePMD-kit (MI355X): model not initialised");
  }
};

// Several models evaluated on the same configuration, and the statistics of
// their spread (model deviation).
class DeepBaseModelDevi {
 public:
  DeepBaseModelDevi() = default;
  virtual ~DeepBaseModelDevi() = default;

  double cutoff() const { return first().cutoff(); }
  int numb_types() const { return first().numb_types(); }
  int numb_types_spin() const { return first().numb_types_spin(); }
  int dim_fparam() const { return first().dim_fparam(); }
  int dim_aparam() const { return first().dim_aparam(); }
  bool is_aparam_nall() const { return false; }
  void get_type_map(std::string& type_map) const { first().get_type_map(type_map); }

  // dener = mean over models of all_energy
  template <typename VALUETYPE>
  void compute_avg(VALUETYPE& dener, const std::vector<VALUETYPE>& all_energy) {
    if (all_energy.empty()) throw deepmd_exception("compute_avg: no models");
    VALUETYPE s = 0;
    for (const VALUETYPE& e : all_energy) s += e;
    dener = s / (VALUETYPE)all_energy.size();
  }
  // avg[j] = mean over models k of xx[k][j]
  template <typename VALUETYPE>
  void compute_avg(std::vector<VALUETYPE>& avg, const std::vector<std::vector<VALUETYPE>>& xx) {
    if (xx.empty()) throw deepmd_exception("compute_avg: no models");
    avg.assign(xx[0].size(), (VALUETYPE)0);
    for (const auto& x : xx) {
      if (x.size() != avg.size()) throw deepmd_exception("compute_avg: models differ in size");
      for (size_t j = 0; j < avg.size(); ++j) avg[j] += x[j];
    }
    for (VALUETYPE& a : avg) a /= (VALUETYPE)xx.size();
  }
  // std[i] = sqrt(mean over models of sum over d < stride of
  //               (xx[k][i*stride+d] - avg[i*stride+d])^2)
  template <typename VALUETYPE>
  void compute_std(std::vector<VALUETYPE>& std, const std::vector<VALUETYPE>& avg,
                   const std::vector<std::vector<VALUETYPE>>& xx, const int& stride) {
    if (xx.empty() || stride <= 0) throw deepmd_exception("compute_std: no models or bad stride");
    const size_t n = avg.size() / (size_t)stride;
    std.assign(n, (VALUETYPE)0);
    for (size_t i = 0; i < n; ++i) {
      VALUETYPE s = 0;
      for (const auto& x : xx)
        for (int d = 0; d < stride; ++d) {
          const VALUETYPE v = x[i * stride + d] - avg[i * stride + d];
          s += v * v;
        }
      std[i] = std::sqrt(s / (VALUETYPE)xx.size());
    }
  }
  // std[i] /= |avg_i| + eps, |avg_i| the norm of avg[i*stride .. +stride)
  template <typename VALUETYPE>
  void compute_relative_std(std::vector<VALUETYPE>& std, const std::vector<VALUETYPE>& avg,
                            const VALUETYPE eps, const int& stride) {
    for (size_t i = 0; i < std.size(); ++i) {
      VALUETYPE s = 0;
      for (int d = 0; d < stride; ++d) s += avg[i * stride + d] * avg[i * stride + d];
      std[i] /= std::sqrt(s) + eps;
    }
  }
  template <typename VALUETYPE>
  void compute_std_f(std::vector<VALUETYPE>& std, const std::vector<VALUETYPE>& avg,
                     const std::vector<std::vector<VALUETYPE>>& xx) {
    compute_std(std, avg, xx, 3);
  }
  template <typename VALUETYPE>
  void compute_relative_std_f(std::vector<VALUETYPE>& std, const std::vector<VALUETYPE>& avg,
                              const VALUETYPE eps) {
    compute_relative_std(std, avg, eps, 3);
  }

  unsigned models() const { return numb_models; }

 protected:
  unsigned numb_models = 0;
  std::vector<std::shared_ptr<DeepBaseModel>> dpbases;

  const DeepBaseModel& first() const {
    if (dpbases.empty()) throw deepmd_exception("DeePMD-kit (MI355X): no models initialised");
    return *dpbases[0];
  }
};

}  // namespace deepmd
