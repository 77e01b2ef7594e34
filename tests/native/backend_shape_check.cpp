// Hosts include/deepmd_amd/DeepPotBackendAMD.h under the interface of the
// reference's backend base. `refshape` below declares, for this check only,
// the virtual members of deepmd::DeepPotBackend with the signatures of
// deepmd-op/overlays/api_cc/include/DeepPot.h:23-155 (init, the four
// computew, the two computew_mixed_type, the charge_spin forms that default
// to them) and :395-445 (the device entries), and the model metadata that
// DeepPotPTExpt.h:103-154 implements for upstream's DeepBaseModelBackend;
// InputNlist carries the fields pair_deepmd.cpp:356-363 sets. DeepPotAMD is
// then declared exactly as a maintainer would declare it inside upstream's
// api_cc: the translation unit compiles (with -Wall -Werror) only if every
// pure virtual is implemented with a matching signature, and the object can
// be created only if none is left abstract.
//
// Modes:
//   backend_shape_check shape
//       compile-and-construct check (no GPU, no model)
//   backend_shape_check run <model> <input>
//       every computew form through a refshape::DeepPotBackend& on one frame
//       (input as facade_check.cpp reads it); prints "E <hex>" (standalone,
//       double), "EF <hex>" (standalone, float), "E2 <hex> <hex>" (two frames
//       of computew_mixed_type), "ENL <hex>" (LAMMPS list of the input taken
//       as an open system), "META <type_map>"
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "deepmd_amd/DeepPotBackendAMD.h"

namespace refshape {

class deepmd_exception : public std::runtime_error {
 public:
  explicit deepmd_exception(const std::string& msg) : std::runtime_error(msg) {}
};

struct InputNlist {
  int inum = 0;
  int* ilist = nullptr;
  int* numneigh = nullptr;
  int** firstneigh = nullptr;
  int mask = 0;
  void set_mask(int m) { mask = m; }
};

class DeepPotBackend {
 public:
  virtual ~DeepPotBackend() {}
  virtual void init(const std::string& model, const int& gpu_rank = 0,
                    const std::string& file_content = "") = 0;
  virtual double cutoff() const = 0;
  virtual int numb_types() const = 0;
  virtual int numb_types_spin() const = 0;
  virtual int dim_fparam() const = 0;
  virtual int dim_aparam() const = 0;
  virtual void get_type_map(std::string& type_map) = 0;
  virtual bool is_aparam_nall() const = 0;
  virtual bool has_default_fparam() const = 0;
  virtual void computew(std::vector<double>& ener, std::vector<double>& force,
                        std::vector<double>& virial, std::vector<double>& atom_energy,
                        std::vector<double>& atom_virial, const std::vector<double>& coord,
                        const std::vector<int>& atype, const std::vector<double>& box,
                        const std::vector<double>& fparam, const std::vector<double>& aparam,
                        const bool atomic) = 0;
  virtual void computew(std::vector<double>& ener, std::vector<float>& force,
                        std::vector<float>& virial, std::vector<float>& atom_energy,
                        std::vector<float>& atom_virial, const std::vector<float>& coord,
                        const std::vector<int>& atype, const std::vector<float>& box,
                        const std::vector<float>& fparam, const std::vector<float>& aparam,
                        const bool atomic) = 0;
  virtual void computew(std::vector<double>& ener, std::vector<double>& force,
                        std::vector<double>& virial, std::vector<double>& atom_energy,
                        std::vector<double>& atom_virial, const std::vector<double>& coord,
                        const std::vector<int>& atype, const std::vector<double>& box,
                        const int nghost, const InputNlist& inlist, const int& ago,
                        const std::vector<double>& fparam, const std::vector<double>& aparam,
                        const bool atomic) = 0;
  virtual void computew(std::vector<double>& ener, std::vector<float>& force,
                        std::vector<float>& virial, std::vector<float>& atom_energy,
                        std::vector<float>& atom_virial, const std::vector<float>& coord,
                        const std::vector<int>& atype, const std::vector<float>& box,
                        const int nghost, const InputNlist& inlist, const int& ago,
                        const std::vector<float>& fparam, const std::vector<float>& aparam,
                        const bool atomic) = 0;
  virtual void computew_mixed_type(std::vector<double>& ener, std::vector<double>& force,
                                   std::vector<double>& virial, std::vector<double>& atom_energy,
                                   std::vector<double>& atom_virial, const int& nframes,
                                   const std::vector<double>& coord, const std::vector<int>& atype,
                                   const std::vector<double>& box,
                                   const std::vector<double>& fparam,
                                   const std::vector<double>& aparam, const bool atomic) = 0;
  virtual void computew_mixed_type(std::vector<double>& ener, std::vector<float>& force,
                                   std::vector<float>& virial, std::vector<float>& atom_energy,
                                   std::vector<float>& atom_virial, const int& nframes,
                                   const std::vector<float>& coord, const std::vector<int>& atype,
                                   const std::vector<float>& box, const std::vector<float>& fparam,
                                   const std::vector<float>& aparam, const bool atomic) = 0;
  // charge_spin forms: the reference's defaults forward to the above
  virtual void computew(std::vector<double>& ener, std::vector<double>& force,
                        std::vector<double>& virial, std::vector<double>& atom_energy,
                        std::vector<double>& atom_virial, const std::vector<double>& coord,
                        const std::vector<int>& atype, const std::vector<double>& box,
                        const std::vector<double>& fparam, const std::vector<double>& aparam,
                        const std::vector<double>& charge_spin, const bool atomic) {
    (void)charge_spin;
    computew(ener, force, virial, atom_energy, atom_virial, coord, atype, box, fparam, aparam,
             atomic);
  }
  virtual void computew(std::vector<double>& ener, std::vector<double>& force,
                        std::vector<double>& virial, std::vector<double>& atom_energy,
                        std::vector<double>& atom_virial, const std::vector<double>& coord,
                        const std::vector<int>& atype, const std::vector<double>& box,
                        const int nghost, const InputNlist& inlist, const int& ago,
                        const std::vector<double>& fparam, const std::vector<double>& aparam,
                        const std::vector<double>& charge_spin, const bool atomic) {
    (void)charge_spin;
    computew(ener, force, virial, atom_energy, atom_virial, coord, atype, box, nghost, inlist,
             ago, fparam, aparam, atomic);
  }
  // device entries (defined out of line upstream; not supported by default)
  virtual void compute_edges_gpu(double*, double*, double*, const double*, const int*,
                                 const int*, const double*, const int, const int) {
    throw deepmd_exception("not supported");
  }
  virtual void compute_edges_gpu(double*, double*, double*, const double*, const int*,
                                 const int*, const double*, const int, const int,
                                 const std::vector<double>&, const std::vector<double>&,
                                 const int, const InputNlist*) {
    throw deepmd_exception("not supported");
  }
  virtual void compute_edges_gpu(double*, double*, double*, const double*, const int*,
                                 const int*, const float*, const int, const int,
                                 const std::vector<double>&, const std::vector<double>&,
                                 const int, const InputNlist*) {
    throw deepmd_exception("not supported");
  }
  virtual void compute_canonical_graph_gpu(double*, double*, double*, const std::int64_t*,
                                           const std::uint32_t*, const float*,
                                           const std::int64_t*, const std::int64_t*,
                                           const std::uint32_t*, const int, const int,
                                           const std::int64_t) {
    throw deepmd_exception("not supported");
  }
  virtual bool supports_device_edge_inference() const { return false; }
  virtual bool uses_fp32_edge_vectors() const { return false; }
  virtual bool uses_canonical_graph_inference() const { return false; }
};

}  // namespace refshape

// As a maintainer would declare it inside upstream's api_cc (namespace deepmd
// there; DeepPotBackend / InputNlist / deepmd_exception are upstream's).
class DeepPotAMD final
    : public deepmd_amd::DeepPotBackendAMD<refshape::DeepPotBackend, refshape::InputNlist,
                                           refshape::deepmd_exception> {
 public:
  using DeepPotBackendAMD::DeepPotBackendAMD;
};

int main(int argc, char** argv) {
  if (argc >= 2 && std::string(argv[1]) == "shape") {
    DeepPotAMD b;  // constructible: nothing left abstract
    refshape::DeepPotBackend& base = b;
    std::printf("SHAPE ok edges=%d\n", (int)base.supports_device_edge_inference());
    return 0;
  }
  if (argc < 4 || std::string(argv[1]) != "run") return 2;
  FILE* f = std::fopen(argv[3], "rb");
  if (!f) return 2;
  int n = 0;
  if (std::fread(&n, 4, 1, f) != 1) return 2;
  std::vector<double> coord(3 * (size_t)n), box(9);
  std::vector<int> atype(n);
  if (std::fread(coord.data(), 8, coord.size(), f) != coord.size()) return 2;
  if (std::fread(atype.data(), 4, atype.size(), f) != atype.size()) return 2;
  if (std::fread(box.data(), 8, 9, f) != 9) return 2;
  std::fclose(f);
  try {
    DeepPotAMD backend(argv[2]);
    refshape::DeepPotBackend& dp = backend;
    std::string tm;
    dp.get_type_map(tm);
    std::printf("META %s\n", tm.c_str());
    std::vector<double> e, force, virial, ae, av;
    const std::vector<double> none;
    dp.computew(e, force, virial, ae, av, coord, atype, box, none, none, true);
    std::printf("E %a\n", e.at(0));
    std::vector<float> ff, vf, aef, avf;
    const std::vector<float> cf(coord.begin(), coord.end()), bf(box.begin(), box.end()), nonef;
    dp.computew(e, ff, vf, aef, avf, cf, atype, bf, nonef, nonef, false);
    std::printf("EF %a\n", e.at(0));
    // two frames of the same configuration with per-frame types
    std::vector<double> c2(coord), b2(box);
    c2.insert(c2.end(), coord.begin(), coord.end());
    b2.insert(b2.end(), box.begin(), box.end());
    std::vector<int> t2(atype);
    t2.insert(t2.end(), atype.begin(), atype.end());
    dp.computew_mixed_type(e, force, virial, ae, av, 2, c2, t2, b2, none, none, false);
    std::printf("E2 %a %a\n", e.at(0), e.at(1));
    // LAMMPS path on the input taken as an open system, full list by brute
    // force with a 1 A skin
    const double rc = dp.cutoff() + 1.0;
    std::vector<std::vector<int>> rows(n);
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) {
        if (i == j) continue;
        double r2 = 0;
        for (int c = 0; c < 3; ++c) {
          const double d = coord[3 * j + c] - coord[3 * i + c];
          r2 += d * d;
        }
        if (r2 <= rc * rc) rows[i].push_back(j);
      }
    std::vector<int> ilist(n), numneigh(n);
    std::vector<int*> firstneigh(n);
    for (int i = 0; i < n; ++i) {
      ilist[i] = i;
      numneigh[i] = (int)rows[i].size();
      firstneigh[i] = rows[i].data();
    }
    refshape::InputNlist nl;
    nl.inum = n;
    nl.ilist = ilist.data();
    nl.numneigh = numneigh.data();
    nl.firstneigh = firstneigh.data();
    nl.set_mask(0x3FFFFFFF);
    const std::vector<double> nobox;
    dp.computew(e, force, virial, ae, av, coord, atype, nobox, 0, nl, 0, none, none, false);
    std::printf("ENL %a\n", e.at(0));
  } catch (const std::exception& ex) {
    std::printf("EXC %s\n", ex.what());
    return 3;
  }
  return 0;
}
