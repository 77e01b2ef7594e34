"""Writes the committed golden fixtures from the CPU oracle (run from the
repository root: python tests/golden/make_golden.py). The fixtures pin the
oracle against regressions and give the GPU tests a reference that needs no
CPU evaluation:
  water192.npz  config-0 nlist (int32 [192, 138]), ghost mapping
  water192.json energy, atom energies, forces, virial as hex floats
  cu864.json    sha256 of the sel-overflowed nlist + energy/forces/virial
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from cases import CASES, model_bytes  # noqa: E402
from _pkg import load_oracle  # noqa: E402


def hexes(a):
    return [float(v).hex() for v in np.asarray(a, dtype=np.float64).reshape(-1)]


def main():
    orc = load_oracle()
    for case in ("water192", "cu864"):
        (coord, atype, box), m = CASES[case]()
        mb = model_bytes(m)
        out = orc.Oracle(mb).compute(coord, atype, box)
        nl = out["nlist"].astype(np.int32)
        doc = {"case": case, "natoms": int(len(atype)),
               "model_sha256": hashlib.sha256(mb).hexdigest(),
               "coord_sha256": hashlib.sha256(np.ascontiguousarray(coord).tobytes()).hexdigest(),
               "nlist_sha256": hashlib.sha256(nl.tobytes()).hexdigest(),
               "nall": int(len(out["ext_type"])),
               "energy": float(out["energy"]).hex(),
               "atom_energy": hexes(out["atom_energy"]),
               "force": hexes(out["force"]),
               "virial": hexes(out["virial"])}
        with open(os.path.join(HERE, f"{case}.json"), "w") as f:
            json.dump(doc, f, indent=0)
        if case == "water192":
            np.savez_compressed(os.path.join(HERE, "water192.npz"), nlist=nl,
                                mapping=out["mapping"].astype(np.int32))
        print(case, "E =", out["energy"], "nall =", doc["nall"])


if __name__ == "__main__":
    main()
