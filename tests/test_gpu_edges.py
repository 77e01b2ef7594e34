"""The compute_edges_gpu entry (dp_compute_edges_device[_f32]) against the CPU
oracles: the caller's device edge graph (edge_index [2][nedge]: source row,
destination row; edge_vec = r_source - r_destination), as the reference's
Kokkos pair builds it from LAMMPS' list with skin
(deepmd-op/overlays/lmp/pair_deepmd_kokkos.cpp:586-597).

fp64 bars as test_gpu_parity (energy/atom 1e-10 eV, forces and virials 1e-8);
DPA4C at the reference's mixed-precision limits."""
import importlib

import numpy as np
import pytest

from _pkg import load_dpa4c_oracle
from cases import CASES, model_bytes

pytestmark = pytest.mark.gpu

C4 = load_dpa4c_oracle()


def _edges(orc_mod, coord, atype, box, rcut, skin=1.0, fold=True):
    """Edges of every (local centre, neighbour within rcut + skin) pair, with
    the ghost images either folded onto their owners (single domain) or kept
    as extended nodes after the locals."""
    ext, et, mp = orc_mod.Oracle.ghosts(coord, atype, box, rcut + skin)
    nloc = len(atype)
    off, cand = orc_mod.Oracle.candidates(nloc, ext, et, rcut + skin, "brute")
    dst = np.repeat(np.arange(nloc), np.diff(off))
    j = cand.astype(np.int64)
    src = mp[j] if fold else j
    vec = ext[j] - ext[dst]
    ei = np.ascontiguousarray(np.stack([src, dst]).astype(np.int32))
    return ext, et, mp, ei, vec


def _run(dp, pot, ei, vec, atype_nodes, nloc, nnode, fp32=False):
    hip = importlib.import_module("dpamd.hip")
    nedge = ei.shape[1]
    d_ei = hip.DeviceArray(ei)
    d_vec = hip.DeviceArray(np.ascontiguousarray(vec, np.float32 if fp32 else np.float64))
    d_at = hip.DeviceArray(np.ascontiguousarray(atype_nodes, np.int32))
    ae = hip.DeviceArray(nbytes=8 * max(nloc, 1))
    f, av = hip.DeviceArray(nbytes=24 * nnode), hip.DeviceArray(nbytes=72 * nnode)
    pot.compute_edges_device(ae.ptr, f.ptr, av.ptr, 0, d_at.ptr, d_ei.ptr, d_vec.ptr, nloc,
                             nedge, nnode, fp32=fp32)
    return (ae.to_host(np.float64, (max(nloc, 1),))[:nloc], f.to_host(np.float64, (nnode, 3)),
            av.to_host(np.float64, (nnode, 9)))


@pytest.mark.parametrize("case", ["cu864", "water24_smallbox", "hea1024"])
def test_edges_folded_fp64(dp, orc, case):
    (coord, atype, box), m = CASES[case]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box)
    ext, et, mp, ei, vec = _edges(orc, coord, atype, box, O.m["rcut"])
    n = len(atype)
    pot = dp.DeepPot(file_content=mb)
    ae, f, av = _run(dp, pot, ei, vec, atype, n, n)
    assert np.abs(ae - ref["atom_energy"]).max() <= 1e-10
    assert np.abs(f - ref["force"]).max() <= 1e-8
    assert np.abs(av - ref["atom_virial"]).max() <= 1e-8
    assert np.abs(av.sum(0) - ref["virial"]).max() <= 1e-8
    # the same graph with its edges in another order gives the same numbers
    perm = np.random.default_rng(3).permutation(ei.shape[1])
    ae2, f2, av2 = _run(dp, pot, np.ascontiguousarray(ei[:, perm]), vec[perm], atype, n, n)
    assert np.abs(f2 - f).max() <= 1e-12 and np.abs(ae2 - ae).max() <= 1e-12


def test_edges_extended_nodes_and_fp32_vectors(dp, orc):
    """nall_nodes > nloc (domain-decomposition form): ghost nodes keep their
    forces and atom virials; and fp32 edge vectors, checked against the oracle
    evaluated on the same rounded vectors."""
    (coord, atype, box), m = CASES["hea1024"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ei, vec = _edges(orc, coord, atype, box, O.m["rcut"], fold=False)
    nloc, nall = len(atype), len(et)
    off, cand = O.candidates(nloc, ext, et, O.m["rcut"], "cell")
    nl = O.format_nlist(nloc, ext, et, off, cand)
    ref = O.eval_ext(nloc, ext, et, nl)
    pot = dp.DeepPot(file_content=mb)
    ae, f, av = _run(dp, pot, ei, vec, et, nloc, nall)
    assert np.abs(ae - ref["atom_energy"]).max() <= 1e-10
    assert np.abs(f - ref["force"]).max() <= 1e-8
    assert np.abs(av - ref["atom_virial"]).max() <= 1e-8
    # fp32 vectors: the oracle on extended atoms placed at the rounded vectors
    v32 = vec.astype(np.float32)
    ae3, f3, av3 = _run(dp, pot, ei, v32, et, nloc, nall, fp32=True)
    syn = np.concatenate([np.zeros((nloc, 3)), v32.astype(np.float64)])
    syn_t = np.concatenate([atype, et[ei[0]]]).astype(np.int32)
    offs, cands = O.candidates(nloc, syn, syn_t, O.m["rcut"], "brute")
    # keep only each centre's own edges (every centre sits at the origin)
    own = np.zeros(len(syn_t), np.int64)
    own[nloc:] = ei[1]
    keep = np.ones(len(cands), bool)
    for i in range(nloc):
        seg = slice(offs[i], offs[i + 1])
        keep[seg] = (cands[seg] >= nloc) & (own[cands[seg]] == i)
    counts = np.array([keep[offs[i]:offs[i + 1]].sum() for i in range(nloc)])
    offs2 = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    nl3 = O.format_nlist(nloc, syn, syn_t, offs2, cands[keep].astype(np.int32))
    r3 = O.eval_ext(nloc, syn, syn_t, nl3)
    assert np.abs(ae3 - r3["atom_energy"]).max() <= 1e-10
    f3ref = np.zeros((nall, 3))
    np.add.at(f3ref, np.arange(nloc), r3["force"][:nloc])
    np.add.at(f3ref, ei[0], r3["force"][nloc:])
    assert np.abs(f3 - f3ref).max() <= 1e-8


def test_edges_dpa4c(dp, orc):
    """A DPA4C model through the edge entry point (single domain, folded)."""
    coord, atype, box = dp.systems.bcc_hea(5, 3.2, seed=8)
    m = dp.dpa4c.random_model("hea", seed=309)
    mb = dp.dpa4c.to_bytes(m)
    ref = C4.Dpa4cOracle(mb).compute(coord, atype, box)
    ext, et, mp, ei, vec = _edges(orc, coord, atype, box, m["rcut"])
    n = len(atype)
    pot = dp.DeepPot(file_content=mb)
    ae, f, av = _run(dp, pot, ei, vec, atype, n, n)
    assert np.abs(ae - ref["atom_energy"]).max() <= 2e-5
    df = f - ref["force"]
    assert np.sqrt((df ** 2).mean()) <= 4e-5 and np.abs(df).max() <= 5e-4


def test_edges_bad_source_is_an_error(dp, orc):
    (coord, atype, box), m = CASES["cu864"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ei, vec = _edges(orc, coord, atype, box, O.m["rcut"])
    n = len(atype)
    pot = dp.DeepPot(file_content=mb)
    bad = ei.copy()
    bad[0, 5] = n + 7  # a source node outside the graph
    with pytest.raises(dp.DeepmdException, match="outside"):
        _run(dp, pot, bad, vec, atype, n, n)
    ae, f, av = _run(dp, pot, ei, vec, atype, n, n)  # the handle works normally afterwards
    assert np.isfinite(f).all()


@pytest.mark.parametrize("kind", ["se_e2_a", "dpa4c"])
def test_edges_empty_graph(dp, orc, kind):
    """No edges (isolated atoms): the energies are those of empty
    environments, forces and virials zero."""
    c = np.array([[0, 0, 0], [30, 0, 0], [0, 30, 0]], float)
    t = np.array([0, 1, 2], np.int32)
    b = np.diag([100.0, 100.0, 100.0]).ravel()
    if kind == "se_e2_a":
        mb = model_bytes(CASES["hea1024"]()[1])
        ref = orc.Oracle(mb).compute(c, t, b)
        tol = 1e-10
    else:
        mb = dp.dpa4c.to_bytes(dp.dpa4c.random_model("hea", seed=309))
        ref = C4.Dpa4cOracle(mb).compute(c, t, b)
        tol = 2e-5
    pot = dp.DeepPot(file_content=mb)
    ei = np.zeros((2, 0), np.int32)
    vec = np.zeros((0, 3))
    ae, f, av = _run(dp, pot, ei, vec, t, 3, 3)
    assert np.abs(ae - ref["atom_energy"]).max() <= tol
    assert not f.any() and not av.any()


def test_edges_mixed_precision(dp, orc):
    """A mixed-precision se_e2_a handle through the edge entry point, at the
    reference's mixed-precision limits (energy/atom 2e-5 eV, force RMSE 4e-5
    and max 5e-4 eV/A)."""
    (coord, atype, box), m = CASES["hea1024"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box)
    ext, et, mp, ei, vec = _edges(orc, coord, atype, box, O.m["rcut"])
    n = len(atype)
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    ae, f, av = _run(dp, pot, ei, vec, atype, n, n)
    assert np.abs(ae - ref["atom_energy"]).max() <= 2e-5
    df = f - ref["force"]
    assert np.sqrt((df ** 2).mean()) <= 4e-5 and np.abs(df).max() <= 5e-4
    assert np.abs(df).max() > 0.0  # the fp32 nets ran


def test_edges_then_cached_lammps_list(dp, orc):
    """The edge entry points build their candidates in the buffers that cache
    a LAMMPS list between rebuilds; a list call with ago > 0 after an edge
    call on the same handle must not format the edge graph's candidates
    against the caller's atoms (it re-uploads the caller's list instead)."""
    from cases import lammps_inputs
    (coord, atype, box), m = CASES["water192"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ilist, numneigh, firstneigh = lammps_inputs(O, coord, atype, box)
    nloc, nall = len(atype), len(et)
    pot = dp.DeepPot(file_content=mb)
    e0, f0, v0 = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=0)
    nl0 = pot.stage(dp.STAGE_NLIST, np.int32, (nloc, O.nnei)).copy()
    # an edge call with the same nloc in between
    _, _, _, ei, vec = _edges(orc, coord, atype, box, O.m["rcut"])
    _run(dp, pot, ei, vec, atype, nloc, nloc)
    e1, f1, v1 = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=1)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, (nloc, O.nnei)), nl0)
    assert e1 == e0
    assert np.array_equal(f1, f0) and np.array_equal(v1, v0)
