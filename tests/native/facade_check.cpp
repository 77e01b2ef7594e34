// Drives the C++ façade (include/deepmd_amd/DeepPot.h) like pair_style deepmd
// would: init from a model file, metadata queries, a standalone compute and a
// LAMMPS-list compute. Input: model path and a raw input file
//   int32 natoms; f64 coord[natoms*3]; int32 atype[natoms]; f64 box[9]
// Output (stdout): "E <hex>" then "F <i> <hex> <hex> <hex>" for the first
// atoms, then "ENL <hex>" for the neighbour-list path on the extended system
// built by brute force here. Exit 3 when the façade throws.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "deepmd_amd/DeepPot.h"

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  FILE* f = std::fopen(argv[2], "rb");
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
    deepmd::DeepPot dp(argv[1]);
    std::string tm;
    dp.get_type_map(tm);
    std::printf("META rcut=%g ntypes=%d type_map=%s\n", dp.cutoff(), dp.numb_types(), tm.c_str());
    double e = 0;
    std::vector<double> force, virial, ae, av;
    dp.compute(e, force, virial, ae, av, coord, atype, box);
    std::printf("E %a\n", e);
    for (int i = 0; i < 4 && i < n; ++i)
      std::printf("F %d %a %a %a\n", i, force[3 * i], force[3 * i + 1], force[3 * i + 2]);
    // LAMMPS path: local atoms are the input (already inside a big box here),
    // no ghosts; full list by brute force with a 1 A skin
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
    deepmd::InputNlist nl(n, ilist.data(), numneigh.data(), firstneigh.data());
    nl.set_mask(0x1FFFFFFF);
    double e2 = 0;
    std::vector<double> f2, v2;
    dp.compute(e2, f2, v2, coord, atype, box, 0, nl, 0);
    std::printf("ENL %a\n", e2);
  } catch (const deepmd::deepmd_exception& ex) {
    std::printf("EXC %s\n", ex.what());
    return 3;
  }
  return 0;
}
