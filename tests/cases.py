"""Seeded systems + models shared by the parity tests (small enough for the
CPU oracle to finish in seconds)."""
import numpy as np

from _pkg import load_pkg

dp = load_pkg()


def water192():
    return dp.systems.build(0), dp.model.random_model("water", seed=1000)


def cu_small(n=6):
    # 864 atoms, box 21.69 A > 2*rcut: every atom has 176 neighbours within 8 A
    # and keeps 138 (sel overflow by 38)
    return dp.systems.fcc(n, 3.615, seed=22), dp.model.random_model("cu", seed=1002)


def hea_small(n=8):
    return dp.systems.bcc_hea(n, 3.2, seed=33), dp.model.random_model("hea", seed=1003)


def water_small_box():
    # 8 molecules in 6.21 A: box < 2*rcut, many images of each atom
    return dp.systems.water(2, 6.21, seed=44), dp.model.random_model("water", seed=1004)


def tilted(system, tilt):
    """The same fractional positions in a triclinic cell whose lattice vectors
    (rows of h) are a = (L, 0, 0), b = (xy, L, 0), c = (xz, yz, L), with
    (xy, xz, yz) = tilt * L: LAMMPS' [xx,0,0, xy,yy,0, xz,yz,zz] box."""
    coord, atype, box = system
    H0 = box.reshape(3, 3)
    frac = coord @ np.linalg.inv(H0)
    H = H0.copy()
    H[1, 0], H[2, 0], H[2, 1] = np.asarray(tilt, np.float64) * H0[0, 0]
    return frac @ H, atype, H.reshape(9).copy()


def water192_tric():
    return tilted(dp.systems.build(0), (0.2, -0.15, 0.1)), dp.model.random_model("water", seed=1005)


def cu_tric():
    # 864 atoms with tilts up to a quarter of the edge: the perpendicular
    # heights shrink, still above 2 rcut
    return tilted(dp.systems.fcc(6, 3.615, seed=23), (-0.1, 0.2, 0.25)), \
        dp.model.random_model("cu", seed=1006)


def water_small_tric():
    # 24 atoms in a tilted 6.21 A cell: several images of each atom per
    # direction, along tilted lattice vectors
    return tilted(dp.systems.water(2, 6.21, seed=45), (0.3, 0.25, -0.2)), \
        dp.model.random_model("water", seed=1007)


CASES = {"water192": water192, "cu864": cu_small, "hea1024": hea_small,
         "water24_smallbox": water_small_box, "water192_tric": water192_tric,
         "cu864_tric": cu_tric, "water24_tric": water_small_tric}


# Fitting shapes the fused dE/dD -> dE/dT kernels do not cover: (system, model
# overrides)
FALLBACK_SHAPES = {
    # F0 != 240 with axis 16: D formed inside the first GEMM, dE/dD as a
    # plain product of the library's GEMM, then the axis-16 dE/dT kernel
    "water_f160": ("water192", dict(fit=[160, 160, 160])),
    # axis != 16: D stored by the descriptor kernel, the first layer reads it,
    # dE/dD plain, then the any-axis dE/dT kernel
    "water_axis8_f192": ("water192", dict(axis=8, fit=[192, 192, 192])),
    "cu_axis4_f160": ("cu864", dict(axis=4, fit=[160, 160, 160])),
    # F0 = 240 but axis 32 (no fused kernel), four centre types
    "hea_axis32": ("hea1024", dict(axis=32)),
}
_KIND_OF = {"water192": "water", "cu864": "cu", "hea1024": "hea"}


def fallback_case(name):
    system, over = FALLBACK_SHAPES[name]
    (coord, atype, box), _ = CASES[system]()
    m = dp.model.random_model(_KIND_OF[system], seed=1020, **over)
    return (coord, atype, box), m


def model_bytes(m):
    return dp.model.to_bytes(m)


def lammps_inputs(orc_obj, coord, atype, box, skin=1.0):
    """Extended system + full neighbour list with skin, shaped like LAMMPS'
    (ilist, numneigh, firstneigh) with ghosts after the local atoms."""
    ext, et, mp = orc_obj.ghosts(coord, atype, box, orc_obj.m["rcut"] + skin)
    nloc = len(atype)
    off, cand = orc_obj.candidates(nloc, ext, et, orc_obj.m["rcut"] + skin, "cell")
    # shuffle each list: LAMMPS order is arbitrary
    rng = np.random.default_rng(5)
    firstneigh = []
    for i in range(nloc):
        row = cand[off[i]:off[i + 1]].copy()
        rng.shuffle(row)
        firstneigh.append(row)
    ilist = np.arange(nloc, dtype=np.int32)[::-1].copy()
    firstneigh = [firstneigh[i] for i in ilist]
    numneigh = np.array([len(r) for r in firstneigh], np.int32)
    return ext, et, mp, ilist, numneigh, firstneigh
