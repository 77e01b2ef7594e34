"""Seeded synthetic systems and the counter-based PRNG they are built from.

The PRNG is splitmix64 used counter-style: value(seed, stream, i) is the
splitmix64 finaliser of (key + (i + 1) * golden), key = finaliser of
(seed + stream * 0xD1B54A32D192ED03). Uniforms take the top 53 bits; normals
use Box-Muller on the uniform pair (2i, 2i+1). Everything is vectorised numpy
with wrapping uint64 arithmetic, so the same seed gives the same system on
any host.

The five workloads follow the benchmark configurations: 192-atom water
(64 H2O, 12.42 A), 12,288-atom water (49.68 A), 131,072-atom FCC Cu
(32^3 cells, a = 3.615 A), 128,000-atom BCC high-entropy alloy (40^3 cells,
a = 3.2 A, four species at exactly 25 %) and 393,216-atom water (51^3 sites
with 1,579 seeded vacancies, 157.5 A). Boxes use LAMMPS' row-major
h = [xx,0,0, xy,yy,0, xz,yz,zz] (lammps-deepmd-plugin/src/pair_deepmd.cpp:293-299).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_STREAM = np.uint64(0xD1B54A32D192ED03)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class Stream:
    """Counter-based splitmix64 stream: draws are pure functions of (seed, stream, i)."""

    def __init__(self, seed: int, stream: int = 0):
        with np.errstate(over="ignore"):
            k = np.array([seed], dtype=np.uint64) + np.array([stream], dtype=np.uint64) * _STREAM
            self.key = _mix(k + _GOLDEN)[0]
        self.pos = 0

    def bits(self, n: int) -> np.ndarray:
        i = np.arange(self.pos, self.pos + n, dtype=np.uint64)
        self.pos += n
        with np.errstate(over="ignore"):
            return _mix(self.key + (i + np.uint64(1)) * _GOLDEN)

    def uniform(self, n: int) -> np.ndarray:
        return (self.bits(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, n: int) -> np.ndarray:
        u = self.uniform(2 * n).reshape(n, 2)
        return np.sqrt(-2.0 * np.log1p(-u[:, 0])) * np.cos(2.0 * np.pi * u[:, 1])

    def permutation(self, n: int) -> np.ndarray:
        return np.argsort(self.bits(n), kind="stable")


def cubic_box(edge: float) -> np.ndarray:
    return np.array([edge, 0, 0, 0, edge, 0, 0, 0, edge], dtype=np.float64)


def water(n_side: int, edge: float, seed: int, n_vacancies: int = 0, sigma: float = 0.1,
          r_oh: float = 0.96, angle_deg: float = 104.52):
    """Jittered-lattice water: O = site + N(0, sigma^2); H = O + r_oh * unit vectors
    at the H-O-H angle `angle_deg`. Atom order: all O, then H1/H2 per molecule.
    Types: O = 0, H = 1."""
    st_sites, st_o, st_h = Stream(seed, 1), Stream(seed, 2), Stream(seed, 3)
    a = edge / n_side
    g = np.arange(n_side, dtype=np.float64)
    sites = np.stack(np.meshgrid(g, g, g, indexing="ij"), axis=-1).reshape(-1, 3)
    if n_vacancies:
        keep = np.sort(st_sites.permutation(len(sites))[n_vacancies:])
        sites = sites[keep]
    nmol = len(sites)
    o = (sites + 0.5) * a + sigma * st_o.normal(3 * nmol).reshape(nmol, 3)
    v = st_h.normal(6 * nmol).reshape(nmol, 2, 3)
    u1 = v[:, 0] / np.linalg.norm(v[:, 0], axis=1, keepdims=True)
    p = v[:, 1] - np.sum(v[:, 1] * u1, axis=1, keepdims=True) * u1
    p /= np.linalg.norm(p, axis=1, keepdims=True)
    th = np.deg2rad(angle_deg)
    u2 = np.cos(th) * u1 + np.sin(th) * p
    h = np.stack([o + r_oh * u1, o + r_oh * u2], axis=1).reshape(-1, 3)
    coord = np.concatenate([o, h], axis=0)
    atype = np.concatenate([np.zeros(nmol, np.int32), np.ones(2 * nmol, np.int32)])
    return coord, atype, cubic_box(edge)


def fcc(n_cells: int, a: float, seed: int, sigma: float = 0.05):
    """FCC lattice (4-atom conventional cell) + N(0, sigma^2) displacements, one type."""
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    g = np.arange(n_cells, dtype=np.float64)
    cells = np.stack(np.meshgrid(g, g, g, indexing="ij"), axis=-1).reshape(-1, 1, 3)
    coord = ((cells + basis[None]) * a).reshape(-1, 3)
    coord = coord + sigma * Stream(seed, 1).normal(coord.size).reshape(-1, 3)
    return coord, np.zeros(len(coord), np.int32), cubic_box(n_cells * a)


def bcc_hea(n_cells: int, a: float, seed: int, ntypes: int = 4, sigma: float = 0.05):
    """BCC lattice, species at exactly 1/ntypes each by a seeded permutation."""
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0.5]])
    g = np.arange(n_cells, dtype=np.float64)
    cells = np.stack(np.meshgrid(g, g, g, indexing="ij"), axis=-1).reshape(-1, 1, 3)
    coord = ((cells + basis[None]) * a).reshape(-1, 3)
    n = len(coord)
    coord = coord + sigma * Stream(seed, 1).normal(coord.size).reshape(-1, 3)
    atype = np.repeat(np.arange(ntypes, dtype=np.int32), n // ntypes)
    atype = np.concatenate([atype, np.arange(n - len(atype), dtype=np.int32)])
    atype = atype[Stream(seed, 2).permutation(n)].astype(np.int32)
    return coord, atype, cubic_box(n_cells * a)


def fcc_alloy(cells, a: float, seed: int, ntypes: int = 2, sigma: float = 0.05):
    """FCC supercell of cells = (nx, ny, nz) conventional cells (orthorhombic
    box), species at exactly 1/ntypes each by a seeded permutation, plus
    N(0, sigma^2) displacements."""
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    nx, ny, nz = cells
    grid = np.stack(np.meshgrid(np.arange(nx, dtype=np.float64), np.arange(ny, dtype=np.float64),
                                np.arange(nz, dtype=np.float64), indexing="ij"), axis=-1)
    coord = ((grid.reshape(-1, 1, 3) + basis[None]) * a).reshape(-1, 3)
    n = len(coord)
    coord = coord + sigma * Stream(seed, 1).normal(coord.size).reshape(-1, 3)
    atype = np.repeat(np.arange(ntypes, dtype=np.int32), n // ntypes)
    atype = np.concatenate([atype, np.arange(n - len(atype), dtype=np.int32)])
    atype = atype[Stream(seed, 2).permutation(n)].astype(np.int32)
    box = np.array([nx * a, 0, 0, 0, ny * a, 0, 0, 0, nz * a], dtype=np.float64)
    return coord, atype, box


# DPA4C workloads: Cu-Ni FCC alloys with the atom counts of the reference's
# CuNi-small / -medium / -large runs (data/workload.csv:2-4: 2,016, 31,920 and
# 499,800 atoms = 4 x 8x7x9, 4 x 20x21x19 and 4 x 50x49x51 cells), a = 3.56 A
C4_WORKLOADS = {
    "cuni2k": dict(cells=(8, 7, 9), kind="cuni"),
    "cuni32k": dict(cells=(20, 21, 19), kind="cuni"),
    "cuni500k": dict(cells=(50, 49, 51), kind="cuni"),
}


def build_c4(name: str, seed: int = 5):
    w = C4_WORKLOADS[name]
    return fcc_alloy(w["cells"], 3.56, seed=seed)


# (system builder, model kind) per benchmark configuration
CONFIGS = {
    0: dict(name="water192", kind="water", build=lambda: water(4, 12.42, seed=0)),
    1: dict(name="water12k", kind="water", build=lambda: water(16, 49.68, seed=1)),
    2: dict(name="cu131k", kind="cu", build=lambda: fcc(32, 3.615, seed=2)),
    3: dict(name="hea128k", kind="hea", build=lambda: bcc_hea(40, 3.2, seed=3)),
    4: dict(name="water393k", kind="water", build=lambda: water(51, 157.5, seed=4, n_vacancies=1579)),
}


def build(config: int):
    """(coord [n,3] f64, atype [n] i32, box [9] f64) of benchmark configuration `config`."""
    return CONFIGS[config]["build"]()


def lammps_list(coord, atype, box, cutoff: float):
    """A LAMMPS-style full neighbour list for an orthorhombic periodic box, as
    `pair_style deepmd` hands it to the model: ghost atoms (periodic images
    within `cutoff` of the box, appended after the local atoms) and, for every
    local atom, all other atoms within `cutoff` (rcut + skin), as a CSR
    (offsets [nloc + 1], neighbours). Returns (ext_coord [nall, 3], ext_type
    [nall], nghost, offsets, neighbours). Built with a cell grid, one stencil
    offset at a time, so memory stays at a few candidate arrays."""
    coord = np.ascontiguousarray(coord, np.float64).reshape(-1, 3)
    atype = np.ascontiguousarray(atype, np.int32)
    h = np.asarray(box, np.float64).reshape(3, 3)
    if np.any(np.abs(h - np.diag(np.diag(h))) > 0):
        raise ValueError("lammps_list: orthorhombic boxes only")
    L = np.diag(h)
    if np.any(L <= 2 * cutoff):
        raise ValueError("lammps_list: box edge must exceed twice the cutoff")
    nloc = len(coord)
    x = coord - np.floor(coord / L) * L
    ext, et = [x], [atype]
    for s in np.ndindex(3, 3, 3):
        sh = np.array(s) - 1
        if not sh.any():
            continue
        y = x + sh * L
        keep = np.all((y >= -cutoff) & (y < L + cutoff), axis=1)
        ext.append(y[keep])
        et.append(atype[keep])
    ext = np.concatenate(ext)
    et = np.concatenate(et).astype(np.int32)
    nall = len(ext)
    nc = np.maximum(1, np.floor((L + 2 * cutoff) / cutoff).astype(np.int64))
    cw = (L + 2 * cutoff) / nc
    cidx = np.minimum(((ext + cutoff) / cw).astype(np.int64), nc - 1)
    cell = (cidx[:, 2] * nc[1] + cidx[:, 1]) * nc[0] + cidx[:, 0]
    order = np.argsort(cell, kind="stable")
    ncell = int(nc.prod())
    cnt = np.bincount(cell, minlength=ncell)
    start = np.concatenate([[0], np.cumsum(cnt)])
    ci = cidx[:nloc]
    rc2 = cutoff * cutoff
    pi, pj = [], []
    for o in np.ndindex(3, 3, 3):
        cc = ci + np.array(o) - 1
        ok = np.all((cc >= 0) & (cc < nc), axis=1)
        centres = np.nonzero(ok)[0]
        cid = (cc[ok, 2] * nc[1] + cc[ok, 1]) * nc[0] + cc[ok, 0]
        k = cnt[cid]
        tot = int(k.sum())
        if tot == 0:
            continue
        i = np.repeat(centres, k)
        first = np.repeat(start[cid], k)
        run = np.arange(tot) - np.repeat(np.cumsum(k) - k, k)
        j = order[first + run]
        d = ext[j] - ext[i]
        m = (np.einsum("ij,ij->i", d, d) < rc2) & (j != i)
        pi.append(i[m])
        pj.append(j[m])
    pi = np.concatenate(pi)
    pj = np.concatenate(pj)
    srt = np.lexsort((pj, pi))
    pi, pj = pi[srt], pj[srt]
    off = np.concatenate([[0], np.cumsum(np.bincount(pi, minlength=nloc))]).astype(np.int64)
    return ext, et, nall - nloc, off, pj.astype(np.int32)
