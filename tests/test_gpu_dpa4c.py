"""GPU parity of the DPA4C-Nano path through the C ABI against the fp64 CPU
oracle (oracle/dpa4c_oracle.py).

The HIP path computes the descriptor and the fitting net in fp32, as the
reference does (fp64 energies); the bars are the reference's own
mixed-precision acceptance limits (data/numeric-tolerances.json:3-9): energy
per atom 2e-5 eV, force RMSE 4e-5 eV/A, force max-abs 5e-4 eV/A, stress
max-abs 4e-4 GPa. Edge lists are bit-exact (the same (i, j) sets as the
oracle's brute-force r^2 < rcut^2 search)."""
import importlib
import types

import numpy as np
import pytest
import torch

from _pkg import load_dpa4c_oracle
from cases import lammps_inputs, tilted

pytestmark = pytest.mark.gpu

C4 = load_dpa4c_oracle()
E_TOL = 2e-5        # eV per atom
F_RMSE = 4e-5       # eV/A
F_MAX = 5e-4        # eV/A
S_TOL = 4e-4        # GPa
EV_A3_TO_GPA = 160.21766208


def _systems(dp):
    return {
        "cu256": (dp.systems.fcc(4, 3.615, seed=7), "cu"),
        "hea250": (dp.systems.bcc_hea(5, 3.2, seed=8), "hea"),
        "water192": (dp.systems.build(0), "water"),
        "water24_smallbox": (dp.systems.water(2, 6.21, seed=44), "water"),
        "cu256_tric": (tilted(dp.systems.fcc(4, 3.615, seed=9), (0.15, -0.2, 0.1)), "cu"),
        "water24_tric": (tilted(dp.systems.water(2, 6.21, seed=46), (-0.3, 0.2, 0.25)), "water"),
        # 768 atoms: the edge passes' grids (16 force blocks of 48 nodes, 24
        # moment / gradient blocks of 32) are multiples of the 8 XCDs, so the
        # nodes are walked XCD by XCD (the smaller systems walk a plain stride)
        "cuni768": (dp.systems.fcc_alloy((4, 4, 12), 3.56, seed=10), "cuni"),
    }


def _volume(box):
    return abs(np.linalg.det(np.asarray(box, np.float64).reshape(3, 3)))


def _check(ref, got, n, vol, nforce=None):
    e, f, v, ae, av = got
    assert abs(e - ref["energy"]) / n <= E_TOL, (e, ref["energy"])
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    df = f - ref["force"]
    assert np.sqrt((df ** 2).mean()) <= F_RMSE, np.sqrt((df ** 2).mean())
    assert np.abs(df).max() <= F_MAX, np.abs(df).max()
    if vol is not None:
        assert np.abs(v - ref["virial"]).max() / vol * EV_A3_TO_GPA <= S_TOL
    # the atom virials sum to the virial to fp32 rounding (the standalone
    # path forms them from the two directions of each edge separately)
    np.testing.assert_allclose(av.sum(0), v, atol=1e-6 * max(1.0, np.abs(v).max()))
    if "atom_virial" in ref:
        scale = max(1.0, np.abs(ref["atom_virial"]).max())
        assert np.abs(av - ref["atom_virial"]).max() <= 1e-5 * scale * 50


def _model(dp, kind, seed):
    m = dp.dpa4c.random_model(kind, seed=seed)
    mb = dp.dpa4c.to_bytes(m)
    return m, mb, C4.Dpa4cOracle(mb)


@pytest.mark.parametrize("case", ["cu256", "hea250", "water192", "water24_smallbox",
                                  "cu256_tric", "water24_tric", "cuni768"])
def test_standalone_parity(dp, case):
    (coord, atype, box), kind = _systems(dp)[case]
    m, mb, O = _model(dp, kind, 300)
    ref = O.compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    assert pot.model_kind == dp.MODEL_DPA4C
    got = pot.compute(coord, atype, box, atomic=True)
    n = len(atype)
    _check(ref, got, n, _volume(box))
    # edge lists: the extended atoms are the oracle's, and every centre's
    # neighbour set is exactly the strict-cutoff set
    nall = len(ref["ext_type"])
    ext = pot.stage(dp.STAGE_EXT_COORD, np.float64, (nall, 3))
    assert ext.tobytes() == ref["ext_coord"].tobytes()
    nl = pot.stage(dp.STAGE_NLIST, np.int32, (n, pot.nnei))
    for i in range(n):
        row = nl[i][nl[i] >= 0]
        assert sorted(row.tolist()) == sorted(ref["src"][ref["dst"] == i].tolist()), i
    # the list keeps candidate order over cell-ordered atoms, not distance
    # order: a fresh handle reproduces the list and every output bit for bit
    pot2 = dp.DeepPot(file_content=mb)
    got2 = pot2.compute(coord, atype, box, atomic=True)
    assert np.array_equal(pot2.stage(dp.STAGE_NLIST, np.int32, (n, pot.nnei)), nl)
    for a, b in zip(got, got2):
        assert np.array_equal(np.asarray(a), np.asarray(b))


@pytest.mark.parametrize("ncell,rcut,min_big", [(6, 9.0, 65), (8, 10.5, 129)])
def test_large_cells(dp, ncell, rcut, min_big):
    """Cells of more than 64 and more than 128 atoms (cutoffs of 9 and 10.5 A
    on Cu-Ni, 4 cells per side of 9.8 and 12.4 A): the cell order then ranks
    two or eight records per lane, and the neighbour list walks runs longer
    than a batch. Parity with the oracle, exact edge sets, and a fresh handle
    reproducing the list and every output bit for bit."""
    coord, atype, box = dp.systems.fcc_alloy((ncell, ncell, ncell), 3.56, seed=31)
    m = dp.dpa4c.random_model("cuni", seed=330, rcut=rcut, sel=[300, 300])
    mb = dp.dpa4c.to_bytes(m)
    ref = C4.Dpa4cOracle(mb).compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    got = pot.compute(coord, atype, box, atomic=True)
    n = len(atype)
    _check(ref, got, n, _volume(box))
    # the cells really are that large: bin the extended atoms as the library
    # does (orthorhombic box: cells of (L + 2 rcut) / floor((L + 2 rcut) / rcut))
    nall = len(ref["ext_type"])
    ext = pot.stage(dp.STAGE_EXT_COORD, np.float64, (nall, 3))
    L = np.diag(np.asarray(box, np.float64).reshape(3, 3))
    nc = np.floor((L + 2 * rcut) / (rcut * (1 + 1e-6))).astype(int)
    cell = np.floor((ext + rcut) / ((L + 2 * rcut) / nc)).astype(int)
    cell = np.clip(cell, 0, nc - 1)
    counts = np.bincount((cell[:, 2] * nc[1] + cell[:, 1]) * nc[0] + cell[:, 0])
    assert counts.max() >= min_big, counts.max()
    nl = pot.stage(dp.STAGE_NLIST, np.int32, (n, pot.nnei))
    for i in range(0, n, 7):
        row = nl[i][nl[i] >= 0]
        assert sorted(row.tolist()) == sorted(ref["src"][ref["dst"] == i].tolist()), i
    pot2 = dp.DeepPot(file_content=mb)
    got2 = pot2.compute(coord, atype, box, atomic=True)
    assert np.array_equal(pot2.stage(dp.STAGE_NLIST, np.int32, (n, pot.nnei)), nl)
    for a, b in zip(got, got2):
        assert np.array_equal(np.asarray(a), np.asarray(b))


@pytest.mark.parametrize("case", ["cu256", "hea250", "water24_smallbox", "cuni768"])
def test_forces_with_and_without_atom_virials(dp, case):
    """The standalone force pass scatters each edge's neighbour side in fixed
    point, with or without the atom virials: the forces, energy and virial of
    the two forms agree bit for bit, match the oracle at the reference's
    limits, and the forces of a periodic system sum to zero."""
    (coord, atype, box), kind = _systems(dp)[case]
    m, mb, O = _model(dp, kind, 300)
    pot = dp.DeepPot(file_content=mb)
    e, f, v = pot.compute(coord, atype, box)
    e2, f2, v2, ae, av = pot.compute(coord, atype, box, atomic=True)
    assert e == e2 and np.array_equal(f, f2) and np.array_equal(v, v2)
    n = len(atype)
    _check(O.compute(coord, atype, box), (e, f, v, ae, av), n, _volume(box))
    assert np.abs(f.sum(0)).max() <= 1e-9 * max(1.0, np.abs(f).max())


@pytest.mark.parametrize("case", ["cu256", "hea250", "cuni768"])
def test_moments_and_cotangents(dp, case):
    """Stage parity: the 44 raw sums per atom and their cotangents dE/d(sums)
    against the oracle (fp32 sums of ~80 edges: relative 2e-5 of the largest
    entry of each block)."""
    (coord, atype, box), kind = _systems(dp)[case]
    m, mb, O = _model(dp, kind, 301)
    ref = O.compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    pot.compute(coord, atype, box)
    n = len(atype)
    mom = pot.stage(dp.STAGE_C4_MOMENTS, np.float32, (n, 44)).astype(np.float64)
    cot = pot.stage(dp.STAGE_C4_COTANGENTS, np.float32, (n, 44)).astype(np.float64)
    at = torch.as_tensor(ref["ext_type"], dtype=torch.long)
    ev = torch.as_tensor(ref["edge_vec"])
    src = torch.as_tensor(ref["src"], dtype=torch.long)
    dst = torch.as_tensor(ref["dst"], dtype=torch.long)
    parts = [p.detach().clone().requires_grad_(True) for p in O.moments(ev, src, dst, at, n)]
    scal, vec, ten, ms, ma = parts
    want = np.concatenate([scal.detach().numpy(), vec.detach().numpy().reshape(n, 12),
                           ten.detach().numpy().reshape(n, 20), ms.detach().numpy()[:, None],
                           ma.detach().numpy()[:, None]], 1)
    raw = O.readout(scal, vec, ten, ms, ma, at[:n])
    D = (raw - O.T["mean"]) * O.T["inv_std"]
    E = O.fitting(D, at[:n]).sum()
    grads = torch.autograd.grad(E, parts)
    gwant = np.concatenate([grads[0].numpy(), grads[1].numpy().reshape(n, 12),
                            grads[2].numpy().reshape(n, 20), grads[3].numpy()[:, None],
                            grads[4].numpy()[:, None]], 1)
    for lo, hi in ((0, 8), (8, 20), (20, 40), (40, 42)):
        scale = np.abs(want[:, lo:hi]).max()
        np.testing.assert_allclose(mom[:, lo:hi], want[:, lo:hi], rtol=0, atol=2e-5 * scale)
        gscale = np.abs(gwant[:, lo:hi]).max()
        np.testing.assert_allclose(cot[:, lo:hi], gwant[:, lo:hi], rtol=0, atol=2e-4 * gscale)
    assert np.all(mom[:, 42:] == 0) and np.all(cot[:, 42:] == 0)


def test_open_cluster(dp):
    """box = NULL: a 60-atom alloy cluster; zero net force and torque."""
    rng = np.random.default_rng(12)
    x = rng.uniform(-5.0, 5.0, (60, 3))
    keep = [0]
    for k in range(1, len(x)):
        if np.linalg.norm(x[keep] - x[k], axis=1).min() > 1.8:
            keep.append(k)
    x = x[keep]
    atype = np.arange(len(x)) % 4
    m, mb, O = _model(dp, "hea", 302)
    ref = O.compute(x, atype, None)
    pot = dp.DeepPot(file_content=mb)
    got = pot.compute(x, atype, None, atomic=True)
    _check(ref, got, len(x), None)
    f = got[1]
    assert np.abs(f.sum(0)).max() < 1e-9
    assert np.abs(np.cross(x, f).sum(0)).max() < 1e-3 * np.abs(f).max() * 10


def test_virtual_atoms(dp):
    """Atoms of type -1 are absent: no energy, no force, never a neighbour
    (the oracle gives them no edges and zero energy)."""
    (coord, atype, box), kind = _systems(dp)["hea250"]
    atype = atype.copy()
    atype[[3, 77, 150]] = -1
    m, mb, O = _model(dp, kind, 308)
    ref = O.compute(coord, atype, box)
    assert not np.isin(ref["src"], np.nonzero(atype < 0)[0]).any()
    pot = dp.DeepPot(file_content=mb)
    got = pot.compute(coord, atype, box, atomic=True)
    _check(ref, got, len(atype), _volume(box))
    e, f, v, ae, av = got
    assert np.all(ae[atype < 0] == 0.0) and np.all(f[atype < 0] == 0.0)


@pytest.mark.parametrize("case", ["hea250", "cuni768"])
def test_lammps_path(dp, orc, case):
    """dp_compute_nlist with a DPA4C model: LAMMPS' full list with skin,
    shuffled rows, ghosts after the locals; ghost forces stay in ghost slots."""
    (coord, atype, box), kind = _systems(dp)[case]
    m, mb, O = _model(dp, kind, 303)
    shim = types.SimpleNamespace(ghosts=orc.Oracle.ghosts, candidates=orc.Oracle.candidates,
                                 m={"rcut": m["rcut"]})
    ext, et, mp, ilist, numneigh, firstneigh = lammps_inputs(shim, coord, atype, box)
    nloc, nall = len(atype), len(et)
    # oracle: every (i local, j extended) pair with r^2 < rcut^2
    dst, src = [], []
    for i in range(nloc):
        d = ext - ext[i]
        r2 = d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1] + d[:, 2] * d[:, 2]
        js = np.nonzero((r2 < m["rcut"] ** 2) & (np.arange(nall) != i))[0]
        dst += [i] * len(js)
        src += js.tolist()
    src, dst = np.array(src), np.array(dst)
    ref = O.evaluate_graph(et, src, dst, ext[src] - ext[dst], nloc, nall)
    pot = dp.DeepPot(file_content=mb)
    got = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=0,
                            atomic=True)
    e, f, v, ae, av = got
    _check(ref, (e, f, v, ae[:nloc], av), nloc, _volume(box))
    # the reverse-list gather sums in a fixed order: a second evaluation
    # gives the same bits
    got2 = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=0,
                             atomic=True)
    for a, b in zip(got, got2):
        assert np.asarray(a).tobytes() == np.asarray(b).tobytes()


def _canonical(ref_ext, ref_et, src, dst, dv, nloc, extra=5):
    """Compact canonical graph arrays (the reference's layout) of an edge set
    sorted by destination."""
    nall = len(ref_et)
    order = np.lexsort((src, dst))
    src, dst, dv = src[order], dst[order], dv[order]
    E = len(src)
    storage = E + extra
    drow = np.zeros(nall + 1, np.int64)
    np.add.at(drow, dst + 1, 1)
    drow = np.cumsum(drow)
    sorder = np.argsort(src, kind="stable").astype(np.uint32)
    srow = np.zeros(nall + 1, np.int64)
    np.add.at(srow, src + 1, 1)
    srow = np.cumsum(srow)
    ev = np.zeros((storage, 3), np.float32)
    ev[:E] = dv.astype(np.float32)
    ev[E:] = 1e6  # reserved slots hold garbage: never read as edges
    source = np.zeros(storage, np.uint32)
    source[:E] = src
    sorder_full = np.zeros(storage, np.uint32)
    sorder_full[:E] = sorder
    return dict(atype=ref_et.astype(np.int64), source=source, edge_vec=ev, drow=drow, srow=srow,
                sorder=sorder_full, storage=storage, src=src, dst=dst, nall=nall)


def _run_canonical(dp, pot, g, nloc):
    hip = importlib.import_module("dpamd.hip")
    nall = g["nall"]
    bufs = {k: hip.DeviceArray(np.ascontiguousarray(g[k]))
            for k in ("atype", "source", "edge_vec", "drow", "srow", "sorder")}
    ae, f, av = (hip.DeviceArray(nbytes=8 * max(nloc, 1)), hip.DeviceArray(nbytes=24 * nall),
                 hip.DeviceArray(nbytes=72 * nall))
    pot.compute_canonical_graph_device(ae.ptr, f.ptr, av.ptr, bufs["atype"].ptr,
                                       bufs["source"].ptr, bufs["edge_vec"].ptr,
                                       bufs["drow"].ptr, bufs["srow"].ptr, bufs["sorder"].ptr,
                                       nloc, nall, g["storage"])
    return (ae.to_host(np.float64, (max(nloc, 1),))[:nloc], f.to_host(np.float64, (nall, 3)),
            av.to_host(np.float64, (nall, 9)))


@pytest.mark.parametrize("case", ["cu256", "water24_smallbox"])
def test_canonical_graph(dp, case):
    """dp_compute_canonical_graph_device on the reference's compact canonical
    graph (fp32 edge vectors, int64 types, uint32 sources, two CSR views)
    against the oracle's evaluate_graph on the same fp32 vectors; forces and
    atom virials unfolded over all nodes."""
    (coord, atype, box), kind = _systems(dp)[case]
    m, mb, O = _model(dp, kind, 304)
    base = O.compute(coord, atype, box)
    nloc = len(atype)
    g = _canonical(base["ext_coord"], base["ext_type"], base["src"], base["dst"],
                   base["edge_vec"], nloc)
    ev64 = g["edge_vec"][:len(g["src"])].astype(np.float64)
    ref = O.evaluate_graph(g["atype"], g["src"], g["dst"], ev64, nloc, g["nall"])
    pot = dp.DeepPot(file_content=mb)
    ae, f, av = _run_canonical(dp, pot, g, nloc)
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    df = f - ref["force"]
    assert np.sqrt((df ** 2).mean()) <= F_RMSE and np.abs(df).max() <= F_MAX
    vol = _volume(box)
    assert np.abs(av.sum(0) - ref["virial"]).max() / vol * EV_A3_TO_GPA <= S_TOL
    # folding the ghost slots onto their owners gives the standalone result
    mp = base["mapping"]
    ff = np.zeros((nloc, 3))
    np.add.at(ff, mp, f)
    dff = ff - base["force"]
    assert np.abs(dff).max() <= F_MAX
    # a second call with the same arrays is bit-identical (deterministic)
    ae2, f2, av2 = _run_canonical(dp, pot, g, nloc)
    assert np.array_equal(f2, f) and np.array_equal(av2, av) and np.array_equal(ae2, ae)


def test_canonical_graph_errors(dp):
    """The reference's dimension check, a model of the wrong family, and an
    out-of-range type (flagged by the kernels, which skip it and stay in
    bounds) are reported as errors."""
    (coord, atype, box), kind = _systems(dp)["cu256"]
    m, mb, O = _model(dp, kind, 305)
    base = O.compute(coord, atype, box)
    nloc = len(atype)
    g = _canonical(base["ext_coord"], base["ext_type"], base["src"], base["dst"],
                   base["edge_vec"], nloc)
    pot = dp.DeepPot(file_content=mb)
    bad = dict(g)
    bad["storage"] = 1
    with pytest.raises(dp.DeepmdException, match="invalid compact canonical graph dimensions"):
        _run_canonical(dp, pot, bad, nloc)
    bad = dict(g)
    bad["atype"] = g["atype"].copy()
    bad["atype"][3] = 5
    with pytest.raises(dp.DeepmdException, match="outside the model"):
        _run_canonical(dp, pot, bad, nloc)
    # the handle works normally afterwards
    ae, f, av = _run_canonical(dp, pot, g, nloc)
    assert np.isfinite(f).all()
    sea = dp.DeepPot(file_content=dp.model.to_bytes(dp.model.random_model("cu", seed=1)))
    with pytest.raises(dp.DeepmdException, match="requires a DPA4C model"):
        _run_canonical(dp, sea, g, nloc)


def test_strict_cutoff_and_sel_overflow(dp):
    """A dimer at exactly rcut has no edge, one just inside has two; a sel too
    small for the neighbourhood is an error, never a truncation."""
    m, mb, O = _model(dp, "cu", 306)
    pot = dp.DeepPot(file_content=mb)
    rc = m["rcut"]
    for dx, nedge in ((rc, 0), (np.nextafter(rc, 0.0), 1)):
        x = np.array([[0.0, 0.0, 0.0], [dx, 0.0, 0.0]])
        e, f, v = pot.compute(x, np.array([0, 0]), None)
        nl = pot.stage(dp.STAGE_NLIST, np.int32, (2, pot.nnei))
        assert (nl[0] >= 0).sum() == nedge
        ref = O.compute(x, np.array([0, 0]), None)
        assert abs(e - ref["energy"]) <= 2 * E_TOL
    small = dp.dpa4c.random_model("cu", seed=306, sel=[40])
    pot2 = dp.DeepPot(file_content=dp.dpa4c.to_bytes(small))
    coord, atype, box = dp.systems.fcc(4, 3.615, seed=7)
    with pytest.raises(dp.DeepmdException, match="sel holds"):
        pot2.compute(coord, atype, box)


def test_device_path_matches_host_path(dp):
    """dp_compute_device and its asynchronous form with a DPA4C model give the
    host path's numbers bit for bit."""
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), kind = _systems(dp)["hea250"]
    m, mb, O = _model(dp, kind, 307)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    n = len(atype)
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(atype.astype(np.int32))
    outs = [hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72),
            hip.DeviceArray(nbytes=8 * n), hip.DeviceArray(nbytes=72 * n)]
    for asynchronous in (False, True):
        if asynchronous:
            pot.compute_device_async(dc.ptr, da.ptr, n, box, *[b.ptr for b in outs], ago=0)
            pot.sync()
        else:
            pot.compute_device(dc.ptr, da.ptr, n, box, *[b.ptr for b in outs], ago=0)
        assert outs[0].to_host(np.float64, (1,))[0] == e
        assert np.array_equal(outs[1].to_host(np.float64, (n, 3)), f)
        assert np.array_equal(outs[2].to_host(np.float64, (9,)), v)
        assert np.array_equal(outs[3].to_host(np.float64, (n,)), ae)
        assert np.array_equal(outs[4].to_host(np.float64, (n, 9)), av)


def _nve_c4(dp, dt, steps, temp=300.0):
    hip = importlib.import_module("dpamd.hip")
    acc, ke, kb = 9.648533212e-3, 103.6427, 8.617333262e-5
    coord, atype, box = dp.systems.fcc_alloy((5, 5, 5), 3.56, seed=9)
    n = len(atype)
    pot = dp.DeepPot(file_content=dp.dpa4c.to_bytes(dp.dpa4c.random_model("cuni", seed=400)))
    mass = np.array([63.546, 58.693])[atype][:, None]
    rng = np.random.default_rng(301)
    v = rng.standard_normal((n, 3)) * np.sqrt(kb * temp / (mass * ke))
    v -= (mass * v).sum(0) / mass.sum()
    x = coord.astype(np.float64).copy()
    dc, da = hip.DeviceArray(x), hip.DeviceArray(atype.astype(np.int32))
    de, df, dv = hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72)

    def force(first):
        dc.upload(x)
        pot.compute_device(dc.ptr, da.ptr, n, box, de.ptr, df.ptr, dv.ptr, ago=0 if first else 1)
        return de.to_host(np.float64, (1,))[0], df.to_host(np.float64, (n, 3))

    e, f = force(True)
    etot, fmax = [], 0.0
    for _ in range(steps):
        v += 0.5 * dt * acc * f / mass
        x += dt * v
        e, f = force(False)
        v += 0.5 * dt * acc * f / mass
        fmax = max(fmax, float(np.abs(f).max()))
        etot.append(e + 0.5 * ke * float((mass * v * v).sum()))
    et = np.asarray(etot) / n
    slope = np.polyfit(np.arange(1, steps + 1) * dt * 1e-3, et, 1)[0]
    return slope, float(np.ptp(et)), fmax


def test_nve_drift(dp):
    """NVE energy conservation of the fp32 DPA4C path against the reference's
    mixed-precision limit, total-energy drift <= 6e-6 eV/atom/ps
    (data/numeric-tolerances.json:8). Velocity Verlet is test scaffolding (the
    MD engine's job): 500-atom FCC Cu-Ni from 300 K with zero momentum, 0.2 ps
    through dp_compute_device at dt = 0.5 fs. The seeded random model holds
    the lattice only for a few tenths of a picosecond (then atoms meet at
    distances where its random radial functions give forces of 10-100 eV/A),
    so the window is 0.2 ps. Also at dt = 1 fs: the energy fluctuation must
    fall roughly as dt^2 between the two (integration error, not a noise
    floor from the fp32 kernels; measured ratio ~3.7)."""
    s1, p1, f1 = _nve_c4(dp, 1.0, 200)
    s5, p5, f5 = _nve_c4(dp, 0.5, 400)
    print(f"dpa4c nve: dt 1.0 drift {s1:.2e} spread {p1:.2e}; dt 0.5 drift {s5:.2e} spread "
          f"{p5:.2e} eV/atom(/ps); max |F| {max(f1, f5):.2f}", flush=True)
    assert abs(s5) <= 6e-6
    assert p1 / p5 >= 2.5
