"""GPU parity of the mixed-precision mode (fp32 embedding and fitting nets,
their products on the bf16 matrix cores at fp32 accuracy; fp64 env matrix,
edge gradients, forces, virial and energy sums)
against the fp64 oracle, to the reference's acceptance limits for mixed
precision (data/numeric-tolerances.json:3-9, docs/VALIDATION.md:56-60 of the
reference):

    energy per atom   max abs <= 2e-5 eV
    force             RMSE    <= 4e-5 eV/A,  max abs <= 5e-4 eV/A
    stress            max abs <= 4e-4 GPa    (virial / volume)

The per-atom energies are held to the energy-per-atom limit as well (the
stricter reading). Each case also checks that the mixed result differs from
the fp64 one, so a silent fp64 evaluation cannot pass as mixed.
"""
import numpy as np
import pytest

from cases import CASES, lammps_inputs, model_bytes

pytestmark = pytest.mark.gpu

E_ATOM = 2e-5      # eV
F_RMSE = 4e-5      # eV/A
F_MAX = 5e-4       # eV/A
S_MAX = 4e-4       # GPa
EV_A3_GPA = 160.21766208  # 1 eV/A^3 in GPa


def _volume(box):
    return abs(np.linalg.det(np.asarray(box, np.float64).reshape(3, 3)))


def _check(n, vol, got, ref, label):
    e, f, v = got[:3]
    de = abs(e - ref["energy"]) / n
    df = f - ref["force"]
    rmse = float(np.sqrt((df ** 2).mean()))
    fmax = float(np.abs(df).max())
    smax = float(np.abs(v - ref["virial"]).max() / vol * EV_A3_GPA)
    print(f"{label}: dE/atom {de:.2e} eV, F rmse {rmse:.2e} max {fmax:.2e} eV/A, "
          f"stress {smax:.2e} GPa", flush=True)
    assert de <= E_ATOM
    assert rmse <= F_RMSE
    assert fmax <= F_MAX
    assert smax <= S_MAX
    if len(got) > 3 and "atom_energy" in ref:
        dae = float(np.abs(got[3] - ref["atom_energy"]).max())
        print(f"{label}: atom energy max {dae:.2e} eV", flush=True)
        assert dae <= E_ATOM
    # the fp32 nets really ran
    assert fmax > 0.0 and de + float(np.abs(v - ref["virial"]).max()) > 0.0


@pytest.mark.parametrize("case", list(CASES))
def test_mixed_against_fp64_oracle(dp, orc, case):
    (coord, atype, box), m = CASES[case]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box, want_internals=True)
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    assert pot.info.precision == dp.PREC_MIXED
    got = pot.compute(coord, atype, box, atomic=True)
    # the geometry is fp64 in both modes: neighbour list bit-exact
    nl = pot.stage(dp.STAGE_NLIST, np.int32, ref["nlist"].shape)
    assert np.array_equal(nl, ref["nlist"])
    _check(len(atype), _volume(box), got, ref, case)
    # atom virials sum to the virial; forces sum to zero (fp64 accumulation)
    assert np.abs(got[4].sum(0) - got[2]).max() <= 1e-9 * max(1.0, np.abs(got[2]).max())
    assert np.abs(got[1].sum(0)).max() <= 1e-10 * len(atype)


@pytest.mark.parametrize("case", ["water192", "cu864"])
def test_mixed_stages(dp, orc, case):
    """Descriptor and dE/dD in fp32 against the oracle's fp64 values, relative
    to each array's scale (fp32 has 24 significant bits)."""
    (coord, atype, box), m = CASES[case]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ref = O.compute(coord, atype, box, want_internals=True)
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    pot.keep_stages(True)
    pot.compute(coord, atype, box)
    n = len(atype)
    d = pot.stage(dp.STAGE_DESCRPT, np.float64, (n, O.ndescrpt))
    assert np.abs(d - ref["descrpt"]).max() <= 1e-5 * np.abs(ref["descrpt"]).max()
    dd = pot.stage(dp.STAGE_DEDD, np.float64, (n, O.ndescrpt))
    assert np.abs(dd - ref["dE_dD"]).max() <= 1e-4 * np.abs(ref["dE_dD"]).max()
    eg = pot.stage(dp.STAGE_EDGE_GRAD, np.float64, (n, O.nnei, 3))
    assert np.abs(eg - ref["edge_grad"]).max() <= 1e-4 * np.abs(ref["edge_grad"]).max()


def test_mixed_lammps_path(dp, orc):
    (coord, atype, box), m = CASES["hea1024"]()
    mb = model_bytes(m)
    O = orc.Oracle(mb)
    ext, et, mp, ilist, numneigh, firstneigh = lammps_inputs(O, coord, atype, box)
    nloc, nall = len(atype), len(et)
    off = np.zeros(nloc + 1, np.int64)
    order = np.argsort(ilist)
    rows = [np.sort(firstneigh[k]) for k in order]
    off[1:] = np.cumsum([len(r) for r in rows])
    nl = O.format_nlist(nloc, ext, et, off, np.concatenate(rows).astype(np.int32))
    ref = O.eval_ext(nloc, ext, et, nl)
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    got = pot.compute_nlist(ext, et, box, nall - nloc, ilist, numneigh, firstneigh, ago=0)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl)
    _check(nloc, _volume(box), got, ref, "hea1024/lammps")


def test_mixed_full_size_hea128k(dp, orc):
    """Config 3 at its full size (128,000-atom HEA, the configuration the
    mixed mode is specified for): mixed against this library's fp64 result,
    which the fp64 tests hold to the oracle, to the same limits; the atom
    energies and edge gradients of the first and last 512 centres against
    the fp64 oracle itself (edge gradients to the force limits); and every
    atom's force and atom virial against the oracle's ProdForce / ProdVirial
    and fold of all the mixed run's own edge gradients (fp64 in both modes,
    so to the fp64 bar: the scatter and fold are exact up to fixed-point
    rounding)."""
    from test_gpu_fullsize import _sample, check_assembly, sample_centres
    coord, atype, box = dp.systems.build(3)
    mb = dp.model.to_bytes(dp.model.random_model("hea", seed=1003))
    ref64 = dp.DeepPot(file_content=mb).compute(coord, atype, box, atomic=True)
    ref = {"energy": ref64[0], "force": ref64[1], "virial": ref64[2], "atom_energy": ref64[3]}
    pot = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    pot.keep_stages(True)
    got = pot.compute(coord, atype, box, atomic=True)
    _check(len(atype), _volume(box), got, ref, "hea128k")
    assert np.abs(got[1].sum(0)).max() <= 1e-10 * len(atype)
    O = orc.Oracle(mb)
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    n = len(atype)
    assert np.array_equal(pot.stage(dp.STAGE_NLIST, np.int32, nl.shape), nl)
    idx = sample_centres(n)
    r = _sample(O, ext, et, nl, idx)
    dae = float(np.abs(got[3][idx] - r["atom_energy"]).max())
    eg = check_assembly(dp, O, pot, ext, nl, mp, got[1], got[2], got[4], "hea128k mixed")
    deg = eg[idx] - r["edge_grad"]
    print(f"hea128k sample vs oracle: atom energy max {dae:.2e} eV, edge grad rmse "
          f"{np.sqrt((deg ** 2).mean()):.2e} max {np.abs(deg).max():.2e} eV/A", flush=True)
    assert dae <= E_ATOM
    assert np.sqrt((deg ** 2).mean()) <= F_RMSE and np.abs(deg).max() <= F_MAX
    assert np.abs(deg).max() > 0.0


def test_precision_from_the_model_file(dp):
    """A model file written for mixed precision is evaluated in mixed
    precision by default (as upstream, the precision comes with the model),
    one written for fp64 in fp64, and an explicit precision overrides the
    file's; the two evaluations differ (the fp32 nets really ran)."""
    (coord, atype, box), m = CASES["cu864"]()
    m64 = dict(m, precision="fp64")
    mmx = dict(m, precision="mixed")
    p64 = dp.DeepPot(file_content=model_bytes(m64))
    pmx = dp.DeepPot(file_content=model_bytes(mmx))
    pov = dp.DeepPot(file_content=model_bytes(mmx), precision=dp.PREC_FP64)
    assert p64.info.precision == dp.PREC_FP64 and pov.info.precision == dp.PREC_FP64
    assert pmx.info.precision == dp.PREC_MIXED
    e64, f64, _ = p64.compute(coord, atype, box)
    emx, fmx, _ = pmx.compute(coord, atype, box)
    eov, fov, _ = pov.compute(coord, atype, box)
    assert eov == e64 and np.array_equal(fov, f64)
    assert emx != e64 and abs(emx - e64) / len(atype) <= E_ATOM


def test_mixed_device_entry_point_and_reproducible(dp):
    import importlib
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), m = CASES["cu864"]()
    pot = dp.DeepPot(file_content=model_bytes(m), precision=dp.PREC_MIXED)
    e, f, v = pot.compute(coord, atype, box)
    n = len(atype)
    dc, da = hip.DeviceArray(coord), hip.DeviceArray(atype.astype(np.int32))
    de, df, dv = hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72)
    for ago in (0, 1):
        pot.compute_device(dc.ptr, da.ptr, n, box, de.ptr, df.ptr, dv.ptr, ago=ago)
        hip.synchronize()
        assert de.to_host(np.float64, (1,))[0] == e
        assert df.to_host(np.float64, (n, 3)).tobytes() == f.tobytes()
        assert dv.to_host(np.float64, (9,)).tobytes() == v.tobytes()


def test_fused_input_gradient_four_wave_blocks(dp, orc):
    """A type of 32,768-65,535 rows runs the fused dE/dD -> dE/dT kernels in
    their 64-row (four-wave) form, which none of the benchmark systems
    reaches: FCC Cu of 55,296 atoms (24^3 cells) in fp64 against the oracle
    on the first and last 256 centres (atom energies, edge gradients), and in
    mixed precision against that fp64 result."""
    from test_gpu_fullsize import _sample, sample_centres
    coord, atype, box = dp.systems.fcc(24, 3.615, seed=77)
    n = len(atype)
    assert 32768 <= n < 65536
    mb = dp.model.to_bytes(dp.model.random_model("cu", seed=1077))
    pot = dp.DeepPot(file_content=mb)
    pot.keep_stages(True)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    O = orc.Oracle(mb)
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    idx = sample_centres(n, 256)
    r = _sample(O, ext, et, nl, idx)
    assert np.abs(ae[idx] - r["atom_energy"]).max() <= 1e-10
    eg = pot.stage(dp.STAGE_EDGE_GRAD, np.float64, (n, O.nnei, 3))[idx]
    assert np.abs(eg - r["edge_grad"]).max() <= 1e-11
    mix = dp.DeepPot(file_content=mb, precision=dp.PREC_MIXED)
    got = mix.compute(coord, atype, box, atomic=True)
    _check(n, _volume(box), got, {"energy": e, "force": f, "virial": v, "atom_energy": ae}, "cu55k")
