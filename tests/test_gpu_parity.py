"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Tolerances (fp64, from the benchmark definition): neighbour lists and types
bit-exact; energy per atom <= 1e-10 eV; forces <= 1e-8 eV/A; virial <= 1e-8 eV
(max abs).
"""
import numpy as np
import pytest

from cases import CASES, FALLBACK_SHAPES, fallback_case, lammps_inputs, model_bytes

pytestmark = pytest.mark.gpu

E_TOL = 1e-10   # eV per atom
F_TOL = 1e-8    # eV/A
V_TOL = 1e-8    # eV


def _run(dp, orc, case, keep=False, fused=False):
    (coord, atype, box), m = CASES[case]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box, want_internals=True)
    pot = dp.DeepPot(file_content=mb)
    if keep:
        pot.keep_stages(True)
    if fused:
        # the fused dE/dD -> dE/dT kernel at this size too (by default a
        # system this small takes the plain product and the dE/dT pass)
        pot.set_fused_rows(0)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    return O, ref, pot, (e, f, v, ae, av), (coord, atype, box)


@pytest.mark.parametrize("case", list(CASES))
def test_nlist_bit_exact(dp, orc, case):
    O, ref, pot, _, (coord, atype, box) = _run(dp, orc, case)
    nall = len(ref["ext_type"])
    ext = pot.stage(dp.STAGE_EXT_COORD, np.float64, (nall, 3))
    assert ext.tobytes() == ref["ext_coord"].tobytes(), "extended coordinates differ"
    mp = pot.stage(dp.STAGE_MAPPING, np.int32, (nall,))
    assert np.array_equal(mp, ref["mapping"])
    et = pot.stage(dp.STAGE_EXT_TYPE, np.int32, (nall,))
    assert np.array_equal(et, ref["ext_type"])
    nl = pot.stage(dp.STAGE_NLIST, np.int32, ref["nlist"].shape)
    assert np.array_equal(nl, ref["nlist"])


@pytest.mark.parametrize("fused", [False, True], ids=["plain_dD", "fused_dDdT"])
@pytest.mark.parametrize("case", list(CASES))
def test_energy_force_virial(dp, orc, case, fused):
    O, ref, pot, (e, f, v, ae, av), (coord, atype, box) = _run(dp, orc, case, fused=fused)
    n = len(atype)
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL


@pytest.mark.parametrize("fused", [False, True], ids=["plain_dD", "fused_dDdT"])
@pytest.mark.parametrize("case", ["water192", "cu864"])
def test_stage_parity(dp, orc, case, fused):
    O, ref, pot, (e, f, v, ae, av), (coord, atype, box) = _run(dp, orc, case, keep=True,
                                                                fused=fused)
    n = len(atype)
    d = pot.stage(dp.STAGE_DESCRPT, np.float64, (n, O.ndescrpt))
    np.testing.assert_allclose(d, ref["descrpt"], rtol=0, atol=1e-12)
    dd = pot.stage(dp.STAGE_DEDD, np.float64, (n, O.ndescrpt))
    np.testing.assert_allclose(dd, ref["dE_dD"], rtol=0, atol=1e-11)
    eg = pot.stage(dp.STAGE_EDGE_GRAD, np.float64, (n, O.nnei, 3))
    np.testing.assert_allclose(eg, ref["edge_grad"], rtol=0, atol=1e-11)
    # keeping the edge gradients changes no output
    pot2 = dp.DeepPot(file_content=model_bytes(CASES[case]()[1]))
    if fused:
        pot2.set_fused_rows(0)
    e2, f2, v2, ae2, av2 = pot2.compute(coord, atype, box, atomic=True)
    assert e2 == e and np.array_equal(f2, f) and np.array_equal(v2, v)
    assert np.array_equal(av2, av)
    with pytest.raises(dp.DeepmdException, match="dp_debug_keep"):
        pot2.stage(dp.STAGE_EDGE_GRAD, np.float64, (n, O.nnei, 3))


@pytest.mark.parametrize("case", ["water192", "hea1024", "water192_tric"])
def test_lammps_path(dp, orc, case):
    (coord, atype, box), m = CASES[case]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ilist, numneigh, firstneigh = lammps_inputs(O, coord, atype, box)
    nloc = len(atype)
    nall = len(et)
    off = np.zeros(nloc + 1, np.int64)
    order = np.argsort(ilist)
    rows = [np.sort(firstneigh[k]) for k in order]
    off[1:] = np.cumsum([len(r) for r in rows])
    cand = np.concatenate(rows).astype(np.int32)
    nl = O.format_nlist(nloc, ext, et, off, cand)
    ref = O.eval_ext(nloc, ext, et, nl)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh,
                                        ago=0, atomic=True)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl)
    assert abs(e - ref["energy"]) / nloc <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL
    # ago > 0 reuses the cached list, re-filtered on new positions
    ext2 = ext + 0.01 * np.random.default_rng(1).standard_normal(ext.shape)
    nl2 = O.format_nlist(nloc, ext2, et, off, cand)
    ref2 = O.eval_ext(nloc, ext2, et, nl2)
    e2, f2, v2 = pot.compute_nlist(ext2, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=3)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl2)
    assert abs(e2 - ref2["energy"]) / nloc <= E_TOL
    assert np.abs(f2 - ref2["force"]).max() <= F_TOL


@pytest.mark.parametrize("kind", ["fcc", "bcc"])
def test_nlist_exact_ties(dp, orc, kind):
    """Perfect lattices (no displacement): every neighbour shell is a set of
    exactly equal distances, so the sel order inside a shell is decided by the
    index tie-break alone, and sel truncation (Cu: 176 in range, 138 kept) cuts
    through a tied shell. The GPU list must still equal the oracle's."""
    if kind == "fcc":
        coord, atype, box = dp.systems.fcc(6, 3.615, seed=5, sigma=0.0)
        m = dp.model.random_model("cu", seed=1002)
    else:
        coord, atype, box = dp.systems.bcc_hea(8, 3.2, seed=6, sigma=0.0)
        m = dp.model.random_model("hea", seed=1003)
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    e, f, v = pot.compute(coord, atype, box)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl)
    ref = O.compute(coord, atype, box)
    assert abs(e - ref["energy"]) / len(atype) <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL


@pytest.mark.parametrize("kind", ["water", "cu"])
def test_open_system(dp, orc, kind):
    """An isolated cluster (box = NULL: no periodic images): a water droplet
    cut from the 12k box and an FCC Cu particle whose inner atoms overflow sel.
    The GPU list must equal the oracle's brute-force one bit for bit, E / F /
    V / atom virials must agree, and, the energy being invariant under
    rotations and translations of the whole cluster, the total force and the
    total torque sum(r x F) must vanish."""
    if kind == "water":
        coord, atype, _ = dp.systems.build(1)
        m = dp.model.random_model("water", seed=1001)
    else:
        coord, atype, _ = dp.systems.fcc(8, 3.615, seed=7)
        m = dp.model.random_model("cu", seed=1002)
    centre = coord.mean(0)
    keep = np.linalg.norm(coord - centre, axis=1) < 11.0
    coord = np.ascontiguousarray(coord[keep] - centre)
    atype = np.ascontiguousarray(atype[keep])
    n = len(atype)
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    off, cand = O.candidates(n, coord, atype, O.m["rcut"], "brute")
    nl = O.format_nlist(n, coord, atype, off, cand)
    ref = O.eval_ext(n, coord, atype, nl)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute(coord, atype, None, atomic=True)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl)
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL
    assert np.abs(f.sum(0)).max() <= 1e-9
    assert np.abs(np.cross(coord, f).sum(0)).max() <= 1e-8


def _check_against_oracle(dp, orc, m, coord, atype, box):
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, ref["nlist"].shape), ref["nlist"])
    n = len(atype)
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    return ref


def test_edge_cases(dp, orc):
    """Edge inputs: an empty system, a single atom whose slots are all padding,
    a water model evaluated on oxygen only (one type has no atoms, so its
    fitting net and its pairs are skipped), and a dimer at exactly rcut
    (r^2 == rcut^2 is kept, as the oracle's inclusive test)."""
    cu = dp.model.random_model("cu", seed=1002)
    water = dp.model.random_model("water", seed=1000)
    box = np.diag([30.0, 30.0, 30.0]).reshape(9)
    pot = dp.DeepPot(file_content=model_bytes(cu))
    e, f, v = pot.compute(np.zeros((0, 3)), np.zeros(0, np.int32), box)
    assert e == 0.0 and f.shape == (0, 3) and not np.any(v)
    ref = _check_against_oracle(dp, orc, cu, np.array([[1.0, 2.0, 3.0]]), np.array([0], np.int32),
                                box)
    assert np.all(ref["nlist"] == -1)
    (coord, atype, wbox), _ = CASES["water192"]()
    oxy = atype == 0
    ref = _check_against_oracle(dp, orc, water, np.ascontiguousarray(coord[oxy]),
                                np.ascontiguousarray(atype[oxy]), wbox)
    assert np.all(ref["nlist"][:, 46:] == -1)
    dimer = np.array([[5.0, 5.0, 5.0], [13.0, 5.0, 5.0]])
    ref = _check_against_oracle(dp, orc, cu, dimer, np.array([0, 0], np.int32), box)
    assert ref["nlist"][0, 0] == 1 and ref["nlist"][1, 0] == 0


def test_lammps_path_ghosts_only(dp, orc):
    """A LAMMPS call with no local atoms, only ghosts (a rank whose domain
    is empty), after a full evaluation on the same handle: there are no
    centres, so the embedding forward (which otherwise clears the fixed-point
    sums) does not run, and the ghost slots' forces and atom virials must
    still come back zero, not the previous step's sums."""
    (coord, atype, box), m = CASES["water192"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ilist, numneigh, firstneigh = lammps_inputs(O, coord, atype, box)
    nloc, nall = len(atype), len(et)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh,
                                        ago=0, atomic=True)
    assert np.any(f[nloc:] != 0.0) and np.any(av[nloc:] != 0.0)
    empty = np.zeros(0, np.int32)
    e0, f0, v0, ae0, av0 = pot.compute_nlist(ext, et, box, nall, empty, empty, [], ago=0,
                                             atomic=True)
    assert e0 == 0.0 and f0.shape == (nall, 3) and av0.shape == (nall, 9)
    assert not np.any(f0) and not np.any(v0) and not np.any(ae0) and not np.any(av0)


def test_virtual_atoms(dp, orc):
    (coord, atype, box), m = CASES["water192"]()
    atype = atype.copy()
    atype[[3, 70, 150]] = -1
    mb = model_bytes(m)
    ref = orc.Oracle(mb).compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    assert abs(e - ref["energy"]) / len(atype) <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.all(f[[3, 70, 150]] == 0.0) and np.all(ae[[3, 70, 150]] == 0.0)


@pytest.mark.parametrize("case,mixed", [("cu864", False), ("hea1024", True)])
def test_bitwise_reproducible(dp, case, mixed):
    """Two evaluations give the same bits (fixed-point force sums, fixed
    reduction trees; mixed: four type chains on their own streams)."""
    (coord, atype, box), m = CASES[case]()
    pot = dp.DeepPot(file_content=model_bytes(m), precision=dp.PREC_MIXED if mixed else dp.PREC_FP64)
    r1 = pot.compute(coord, atype, box, atomic=True)
    r2 = pot.compute(coord, atype, box, atomic=True)
    assert r1[0] == r2[0]
    for a, b in zip(r1[1:], r2[1:]):
        assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("mixed", [False, True])
def test_fixed_point_range_guard(dp, mixed):
    """The force stage (both precisions) sums edge forces in 64-bit fixed
    point; an edge gradient large enough to wrap those sums (here: the energy
    head scaled by 1e9) is reported as a capacity error instead of giving
    wrong forces, and the flag does not outlive the evaluation that raised
    it."""
    (coord, atype, box), m = CASES["water192"]()
    m = dict(m)
    fp = m["fit_params"].copy()
    F2 = int(m["fit"][2])
    fp[:, -(F2 + 1):-1] *= 1e9
    m["fit_params"] = fp
    pot = dp.DeepPot(file_content=model_bytes(m), precision=dp.PREC_MIXED if mixed else dp.PREC_FP64)
    with pytest.raises(dp.DeepmdException, match="fixed-point"):
        pot.compute(coord, atype, box)
    # two atoms farther apart than rcut: no edges, nothing to overflow
    e, f, v = pot.compute(np.array([[0.0, 0.0, 0.0], [9.0, 0.0, 0.0]]), np.array([0, 1]), None)
    assert np.all(f == 0.0) and np.isfinite(e)


@pytest.mark.parametrize("fit", [(240, 240, 160), (240, 160, 160), (240, 240, 80)])
def test_fitting_shapes(dp, orc, fit):
    """Fitting nets whose hidden layers are not all square: a non-square layer
    has no residual and no timestep (h = tanh(xW + b)), in the layer before
    the head (the last layer's epilogue with the energy head fused) and in a
    middle layer; widths that are not multiples of the GEMM's 80-column tile
    (160, 80) give other column-block counts for the head's partial energies."""
    coord, atype, box = dp.systems.build(0)
    m = dp.model.random_model("water", seed=1010, fit=list(fit))
    mb = model_bytes(m)
    ref = orc.Oracle(mb).compute(coord, atype, box)
    e, f, v, ae, av = dp.DeepPot(file_content=mb).compute(coord, atype, box, atomic=True)
    n = len(atype)
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL


@pytest.mark.parametrize("name", list(FALLBACK_SHAPES))
@pytest.mark.parametrize("mixed", [False, True])
def test_fitting_fallback_shapes(dp, orc, name, mixed):
    """Fitting shapes the fused dE/dD -> dE/dT kernels do not cover (first
    fitting layer other than 240 wide, or axis other than 16): every output
    against the oracle, in fp64 to the fp64 bar and in mixed precision to the
    reference's mixed-precision limits; the library's own kernels only (no
    vendor BLAS is linked)."""
    from test_gpu_mixed import _check as mixed_check, _volume
    (coord, atype, box), m = fallback_case(name)
    mb = model_bytes(m)
    ref = orc.Oracle(mb).compute(coord, atype, box)
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED if mixed else dp.PREC_FP64)
    got = pot.compute(coord, atype, box, atomic=True)
    n = len(atype)
    if mixed:
        mixed_check(n, _volume(box), got, ref, f"{name} mixed")
        return
    e, f, v, ae, av = got
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL
