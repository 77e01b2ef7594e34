// Hosts the reference pair style's model members on the façade. The two
// structs below declare the members exactly as the reference plugin does
// (lammps-deepmd-plugin/src/pair_base.h:33-36, :61-62 bind a
// deepmd_compat::DeepBaseModel& and a deepmd_compat::DeepBaseModelDevi& in the
// base's constructor; pair_deepmd.h:55-56 declare a deepmd_compat::DeepPot
// and a deepmd_compat::DeepPotModelDevi that the derived constructor hands to
// it), with the headers included by the names the plugin build uses
// (LMPPLUGIN: "DeepBaseModel.h", "DeepPot.h") and `namespace deepmd_compat =
// deepmd;`. Every model call of pair_deepmd.cpp / pair_base.cpp appears below
// with the argument types used there; LAMMPS itself is not needed for that.
//
// Modes:
//   pair_shape_check stats
//       model-deviation statistics on hand-made values against their closed
//       forms (no GPU); exit 0 when they agree
//   pair_shape_check run <model-a> <model-b> <input>
//       init as `pair_style deepmd a b` does, then one step through each
//       branch; prints "E <hex>" (single model), "ENL <hex>", "DEVI_E <hex>
//       <hex>", "DEVI_F <max std_f> <mean std_f>", "DEVI_V <max std_v>";
//       input as facade_check.cpp reads it
#include <cmath>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "DeepBaseModel.h"
#include "DeepPot.h"

namespace deepmd_compat = deepmd;

struct PairDeepBaseModelShape {
  PairDeepBaseModelShape(deepmd_compat::DeepBaseModel& deep_model,
                         deepmd_compat::DeepBaseModelDevi& deep_model_devi)
      : deep_base(deep_model), deep_base_model_devi(deep_model_devi) {}
  void print_summary(const std::string pre) const { deep_base.print_summary(pre); }
  std::string get_file_content(const std::string& model) {
    std::string file_content;
    deepmd_compat::read_file_to_string(model, file_content);
    return file_content;
  }
  std::vector<std::string> get_file_content(const std::vector<std::string>& models) {
    std::vector<std::string> out;
    for (const auto& m : models) out.push_back(get_file_content(m));
    return out;
  }
  deepmd_compat::DeepBaseModel& deep_base;
  deepmd_compat::DeepBaseModelDevi& deep_base_model_devi;
  double cutoff = 0;
  int numb_types = 0, numb_types_spin = 0, dim_fparam = 0, dim_aparam = 0, dim_chg_spin = 0;
};

struct PairDeepMDShape : PairDeepBaseModelShape {
  PairDeepMDShape() : PairDeepBaseModelShape(deep_pot, deep_pot_model_devi) {}
  deepmd_compat::DeepPot deep_pot;
  deepmd_compat::DeepPotModelDevi deep_pot_model_devi;

  // pair_deepmd.cpp:665-697 (coeff / settings)
  void settings(const std::vector<std::string>& models) {
    if (models.size() == 1) {
      deep_pot.init(models[0], 0, get_file_content(models[0]));
      cutoff = deep_pot.cutoff();
      numb_types = deep_pot.numb_types();
      numb_types_spin = deep_pot.numb_types_spin();
      dim_fparam = deep_pot.dim_fparam();
      dim_aparam = deep_pot.dim_aparam();
      dim_chg_spin = deep_pot.dim_chg_spin();
    } else {
      deep_pot.init(models[0], 0, get_file_content(models[0]));
      deep_pot_model_devi.init(models, 0, get_file_content(models));
      cutoff = deep_pot_model_devi.cutoff();
      numb_types = deep_pot_model_devi.numb_types();
      numb_types_spin = deep_pot_model_devi.numb_types_spin();
      dim_fparam = deep_pot_model_devi.dim_fparam();
      dim_aparam = deep_pot_model_devi.dim_aparam();
      dim_chg_spin = deep_pot_model_devi.dim_chg_spin();
      if (cutoff != deep_pot.cutoff() || numb_types != deep_pot.numb_types() ||
          numb_types_spin != deep_pot.numb_types_spin() || dim_fparam != deep_pot.dim_fparam() ||
          dim_aparam != deep_pot.dim_aparam() || dim_chg_spin != deep_pot.dim_chg_spin())
        throw deepmd_compat::deepmd_exception("model metadata differ");
    }
    // pair_deepmd.cpp:881-886
    std::vector<double> charge_spin;
    deep_pot.set_charge_spin(charge_spin);
    if (models.size() > 1) deep_pot_model_devi.set_charge_spin(charge_spin);
    // pair_deepmd.cpp:1000
    std::string type_map_str;
    deep_pot.get_type_map(type_map_str);
    print_summary("  ");
  }
};

static int fail(const char* what) {
  std::printf("FAIL %s\n", what);
  return 1;
}

static int stats_mode() {
  deepmd_compat::DeepPotModelDevi devi;  // statistics need no loaded model
  // two models, two atoms: forces (1,2,2) / (3,2,2) and (0,0,0) / (0,0,4)
  std::vector<std::vector<double>> all_force = {{1, 2, 2, 0, 0, 0}, {3, 2, 2, 0, 0, 4}};
  std::vector<double> avg, std_f;
  devi.compute_avg(avg, all_force);
  const std::vector<double> avg_ref = {2, 2, 2, 0, 0, 2};
  if (avg != avg_ref) return fail("compute_avg");
  devi.compute_std_f(std_f, avg, all_force);
  // atom 0: deviations (-1,0,0), (1,0,0) -> sqrt((1 + 1) / 2) = 1; atom 1: 2
  if (std_f.size() != 2 || std::fabs(std_f[0] - 1.0) > 1e-15 || std::fabs(std_f[1] - 2.0) > 1e-15)
    return fail("compute_std_f");
  devi.compute_relative_std_f(std_f, avg, 0.5);
  // |avg_0| = sqrt(12), |avg_1| = 2
  if (std::fabs(std_f[0] - 1.0 / (std::sqrt(12.0) + 0.5)) > 1e-15 ||
      std::fabs(std_f[1] - 2.0 / 2.5) > 1e-15)
    return fail("compute_relative_std_f");
  // virials with stride 1: component-wise spread
  std::vector<std::vector<double>> all_v = {{1, 0, 0, 0, 1, 0, 0, 0, 1}, {3, 0, 0, 0, 1, 0, 0, 0, -1}};
  std::vector<double> avg_v, std_v;
  devi.compute_avg(avg_v, all_v);
  devi.compute_std(std_v, avg_v, all_v, 1);
  if (std_v.size() != 9 || std_v[0] != 1.0 || std_v[4] != 0.0 || std_v[8] != 1.0)
    return fail("compute_std stride 1");
  devi.compute_relative_std(std_v, avg_v, 1.0, 1);
  if (std::fabs(std_v[0] - 1.0 / 3.0) > 1e-15 || std_v[8] != 1.0) return fail("compute_relative_std");
  double e = 0;
  devi.compute_avg(e, std::vector<double>{1.0, 2.0, 6.0});
  if (e != 3.0) return fail("compute_avg energy");
  std::printf("STATS OK\n");
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && std::string(argv[1]) == "stats") return stats_mode();
  if (argc < 5 || std::string(argv[1]) != "run") return 2;
  FILE* f = std::fopen(argv[4], "rb");
  if (!f) return 2;
  int n = 0;
  if (std::fread(&n, 4, 1, f) != 1) return 2;
  std::vector<double> dcoord(3 * (size_t)n), dbox(9);
  std::vector<int> dtype(n);
  if (std::fread(dcoord.data(), 8, dcoord.size(), f) != dcoord.size()) return 2;
  if (std::fread(dtype.data(), 4, dtype.size(), f) != dtype.size()) return 2;
  if (std::fread(dbox.data(), 8, 9, f) != 9) return 2;
  std::fclose(f);
  try {
    PairDeepMDShape single, multi;
    single.settings({argv[2]});
    multi.settings({argv[2], argv[3]});
    std::vector<double> fparam, daparam, charge_spin;
    // single model, no list (pair_deepmd.cpp:594)
    double dener = 0;
    std::vector<double> dforce, dvirial, deatom, dvatom;
    single.deep_pot.compute(dener, dforce, dvirial, dcoord, dtype, dbox);
    std::printf("E %a\n", dener);
    // single model with a LAMMPS list, plain and per-atom (pair_deepmd.cpp:356-384)
    const double rc = single.cutoff + 1.0;
    std::vector<std::vector<int>> rows(n);
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) {
        if (i == j) continue;
        double r2 = 0;
        for (int c = 0; c < 3; ++c) {
          const double d = dcoord[3 * j + c] - dcoord[3 * i + c];
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
    int nswap = 0, world = 0;
    deepmd_compat::InputNlist lmp_list(n, ilist.data(), numneigh.data(), firstneigh.data(), nswap,
                                       nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &world,
                                       1);
    lmp_list.set_mask(0x1FFFFFFF);
    const int nghost = 0, ago = 0;
    single.deep_pot.compute(dener, dforce, dvirial, dcoord, dtype, dbox, nghost, lmp_list, ago,
                            fparam, daparam, charge_spin);
    std::printf("ENL %a\n", dener);
    single.deep_pot.compute(dener, dforce, dvirial, deatom, dvatom, dcoord, dtype, dbox, nghost,
                            lmp_list, 1, fparam, daparam, charge_spin);
    // model deviation (pair_deepmd.cpp:418-446, :490-535)
    std::vector<double> all_energy;
    std::vector<std::vector<double>> all_force, all_virial, all_atom_energy, all_atom_virial;
    multi.deep_pot_model_devi.compute(all_energy, all_force, all_virial, dcoord, dtype, dbox,
                                      nghost, lmp_list, ago, fparam, daparam, charge_spin);
    multi.deep_pot_model_devi.compute(all_energy, all_force, all_virial, all_atom_energy,
                                      all_atom_virial, dcoord, dtype, dbox, nghost, lmp_list, 1,
                                      fparam, daparam, charge_spin);
    std::printf("DEVI_E %a %a\n", all_energy[0], all_energy[1]);
    if (all_energy[0] != dener) return fail("first model of the deviation != single model");
    std::vector<double> std_f, tmp_avg_f;
    multi.deep_pot_model_devi.compute_avg(tmp_avg_f, all_force);
    multi.deep_pot_model_devi.compute_std_f(std_f, tmp_avg_f, all_force);
    double fmax = 0, fmean = 0;
    for (int i = 0; i < n; ++i) {
      fmax = std::max(fmax, std_f[i]);
      fmean += std_f[i] / n;
    }
    std::printf("DEVI_F %a %a\n", fmax, fmean);
    multi.deep_pot_model_devi.compute_relative_std_f(std_f, tmp_avg_f, 0.1);
    std::vector<std::vector<double>> all_virial_1(2, std::vector<double>(9));
    for (int k = 0; k < 2; ++k)
      for (int q = 0; q < 9; ++q) all_virial_1[k][q] = all_virial[k][q] / n;
    std::vector<double> avg_virial, std_virial;
    multi.deep_pot_model_devi.compute_avg(avg_virial, all_virial_1);
    multi.deep_pot_model_devi.compute_std(std_virial, avg_virial, all_virial_1, 1);
    multi.deep_pot_model_devi.compute_relative_std(std_virial, avg_virial, 0.1, 1);
    double vmax = 0;
    for (double v : std_virial) vmax = std::max(vmax, v);
    std::printf("DEVI_V %a\n", vmax);
  } catch (const deepmd_compat::deepmd_exception& ex) {
    std::printf("EXC %s\n", ex.what());
    return 3;
  }
  return 0;
}
