"""GPU checks at the benchmark sizes and through every entry point.

Full-size parity: neighbour lists bit-exact against the oracle's cell list,
full E/F/V against the oracle on the 12,288-atom water box, and on the large
systems the atom energies and edge gradients of the first and last 512
centres against the oracle, every atom's force and atom virial against the
oracle's own ProdForce / ProdVirial and ghost fold applied to all of the
GPU's edge gradients (so a mis-routed scatter target, a wrong fold or an
index overflow fails at full size), plus size-independent properties (sum of
forces, virial symmetry, sum of atom virials). Tolerances as in
test_gpu_parity.py (fp64: 1e-10 eV/atom, 1e-8 eV/A, 1e-8 eV)."""
import hashlib
import importlib
import json
import os
import subprocess

import numpy as np
import pytest

from cases import CASES, model_bytes
from test_native import build_backend_shape, build_facade, build_pair_shape, write_input

pytestmark = pytest.mark.gpu

E_TOL, F_TOL, V_TOL = 1e-10, 1e-8, 1e-8
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KIND = {1: "water", 2: "cu", 3: "hea", 4: "water"}


@pytest.mark.parametrize("case", ["water192", "cu864"])
def test_gpu_against_golden(dp, case):
    with open(os.path.join(GOLDEN, f"{case}.json")) as f:
        doc = json.load(f)
    unhex = lambda v: np.array([float.fromhex(x) for x in v])  # noqa: E731
    (coord, atype, box), m = CASES[case]()
    pot = dp.DeepPot(file_content=model_bytes(m))
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    nl = pot.stage(dp.STAGE_NLIST, np.int32, (len(atype), pot.nnei))
    assert hashlib.sha256(nl.tobytes()).hexdigest() == doc["nlist_sha256"]
    assert abs(e - float.fromhex(doc["energy"])) / len(atype) <= E_TOL
    assert np.abs(ae - unhex(doc["atom_energy"])).max() <= E_TOL
    assert np.abs(f.reshape(-1) - unhex(doc["force"])).max() <= F_TOL
    assert np.abs(v - unhex(doc["virial"])).max() <= V_TOL


def test_device_entry_point_matches_host_entry_point(dp):
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), m = CASES["hea1024"]()
    pot = dp.DeepPot(file_content=model_bytes(m))
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    n = len(atype)
    dc, da = hip.DeviceArray(coord), hip.DeviceArray(atype.astype(np.int32))
    de, df, dv = hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72)
    dae, dav = hip.DeviceArray(nbytes=8 * n), hip.DeviceArray(nbytes=72 * n)
    for ago in (0, 1):
        pot.compute_device(dc.ptr, da.ptr, n, box, de.ptr, df.ptr, dv.ptr, dae.ptr, dav.ptr, ago=ago)
        hip.synchronize()
        assert de.to_host(np.float64, (1,))[0] == e
        assert df.to_host(np.float64, (n, 3)).tobytes() == f.tobytes()
        assert dv.to_host(np.float64, (9,)).tobytes() == v.tobytes()
        assert dae.to_host(np.float64, (n,)).tobytes() == ae.tobytes()
        assert dav.to_host(np.float64, (n, 9)).tobytes() == av.tobytes()


def test_cpp_facade_on_gpu(dp, orc, tmp_path):
    exe = build_facade(tmp_path)
    (coord, atype, box), m = CASES["water192"]()
    mpath = tmp_path / "m.dp"
    dp.model.write_model(str(mpath), m)
    write_input(tmp_path / "in.bin", coord, atype, box)
    r = subprocess.run([str(exe), str(mpath), str(tmp_path / "in.bin")], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = {ln.split()[0]: ln.split()[1:] for ln in r.stdout.splitlines()}
    assert "type_map=O H" in r.stdout
    O = orc.Oracle(model_bytes(m))
    ref = O.compute(coord, atype, box)
    assert abs(float.fromhex(lines["E"][0]) - ref["energy"]) / len(atype) <= E_TOL
    # neighbour-list path on the same coordinates taken as an open system
    off, cand = O.candidates(len(atype), coord, atype, O.m["rcut"], "brute")
    nl = O.format_nlist(len(atype), coord, atype, off, cand)
    ref2 = O.eval_ext(len(atype), coord, atype, nl)
    assert abs(float.fromhex(lines["ENL"][0]) - ref2["energy"]) / len(atype) <= E_TOL


def test_pair_style_shape_on_gpu(dp, orc, tmp_path):
    """The pair style's model members driven through every branch it takes
    (single model with and without a list, model deviation of two models):
    energies against the oracle, deviation statistics against numpy on the
    oracle's forces and virials of both models."""
    exe = build_pair_shape(tmp_path)
    (coord, atype, box), m = CASES["water192"]()
    m2 = dict(m)
    m2["fit_params"] = m["fit_params"] * 1.01
    pa, pb = tmp_path / "a.dp", tmp_path / "b.dp"
    dp.model.write_model(str(pa), m)
    dp.model.write_model(str(pb), m2)
    write_input(tmp_path / "in.bin", coord, atype, box)
    r = subprocess.run([str(exe), "run", str(pa), str(pb), str(tmp_path / "in.bin")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = {ln.split()[0]: ln.split()[1:] for ln in r.stdout.splitlines() if ln[:1].isupper()}
    n = len(atype)
    ref = orc.Oracle(model_bytes(m)).compute(coord, atype, box)
    assert abs(float.fromhex(out["E"][0]) - ref["energy"]) / n <= E_TOL
    # list path: the input taken as an open system (no ghosts)
    res = []
    for mm in (m, m2):
        O = orc.Oracle(model_bytes(mm))
        off, cand = O.candidates(n, coord, atype, O.m["rcut"], "brute")
        res.append(O.eval_ext(n, coord, atype, O.format_nlist(n, coord, atype, off, cand)))
    assert abs(float.fromhex(out["ENL"][0]) - res[0]["energy"]) / n <= E_TOL
    ea, eb = (float.fromhex(x) for x in out["DEVI_E"])
    assert abs(ea - res[0]["energy"]) / n <= E_TOL and abs(eb - res[1]["energy"]) / n <= E_TOL
    fs = np.stack([x["force"] for x in res])
    std_f = np.sqrt(((fs - fs.mean(0)) ** 2).sum(2).mean(0))
    fmax, fmean = (float.fromhex(x) for x in out["DEVI_F"])
    assert fmax == pytest.approx(std_f.max(), rel=1e-6) and fmean == pytest.approx(std_f.mean(), rel=1e-6)
    vs = np.stack([x["virial"] for x in res]) / n
    assert float.fromhex(out["DEVI_V"][0]) == pytest.approx(
        (np.sqrt(((vs - vs.mean(0)) ** 2).mean(0)) / (np.abs(vs.mean(0)) + 0.1)).max(), rel=1e-6)


def test_backend_adapter_on_gpu(dp, orc, tmp_path):
    """Every computew form of the backend adapter, called through the
    reference's backend interface, against the oracle: standalone in double
    and float, two frames with per-frame types, and the LAMMPS list."""
    exe = build_backend_shape(tmp_path)
    (coord, atype, box), m = CASES["water192"]()
    mpath = tmp_path / "m.dp"
    dp.model.write_model(str(mpath), m)
    write_input(tmp_path / "in.bin", coord, atype, box)
    r = subprocess.run([str(exe), "run", str(mpath), str(tmp_path / "in.bin")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = {ln.split()[0]: ln.split()[1:] for ln in r.stdout.splitlines()}
    assert out["META"] == ["O", "H"]
    n = len(atype)
    O = orc.Oracle(model_bytes(m))
    ref = O.compute(coord, atype, box)
    assert abs(float.fromhex(out["E"][0]) - ref["energy"]) / n <= E_TOL
    # float coordinates: the configuration rounded to fp32 (energy to 1e-4 eV/atom)
    assert abs(float.fromhex(out["EF"][0]) - ref["energy"]) / n <= 1e-4
    e2 = [float.fromhex(x) for x in out["E2"]]
    assert e2[0] == e2[1] and abs(e2[0] - ref["energy"]) / n <= E_TOL
    off, cand = O.candidates(n, coord, atype, O.m["rcut"], "brute")
    ref2 = O.eval_ext(n, coord, atype, O.format_nlist(n, coord, atype, off, cand))
    assert abs(float.fromhex(out["ENL"][0]) - ref2["energy"]) / n <= E_TOL


def _full(dp, orc, cfg):
    coord, atype, box = dp.systems.build(cfg)
    mb = dp.model.to_bytes(dp.model.random_model(KIND[cfg], seed=1000 + cfg))
    O = orc.Oracle(mb)
    pot = dp.DeepPot(file_content=mb)
    pot.keep_stages(True)
    e, f, v, ae, av = pot.compute(coord, atype, box, atomic=True)
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    gnl = pot.stage(dp.STAGE_NLIST, np.int32, nl.shape)
    assert np.array_equal(gnl, nl), "full-size neighbour list differs"
    return O, pot, (coord, atype, box), (e, f, v, ae, av), (ext, et, mp, nl)


def test_full_water12k_all_outputs(dp, orc):
    O, _, (coord, atype, box), (e, f, v, ae, av), _ = _full(dp, orc, 1)
    ref = O.compute(coord, atype, box)
    n = len(atype)
    assert abs(e - ref["energy"]) / n <= E_TOL
    assert np.abs(ae - ref["atom_energy"]).max() <= E_TOL
    assert np.abs(f - ref["force"]).max() <= F_TOL
    assert np.abs(v - ref["virial"]).max() <= V_TOL
    assert np.abs(av - ref["atom_virial"]).max() <= V_TOL


def _sample(O, ext, et, nl, idx):
    """Oracle evaluation of the centres idx alone: copies of them are put
    first in the extended arrays and their neighbour indices shifted past the
    copies, so eval_ext sees them as its K local atoms."""
    K = len(idx)
    ext2 = np.concatenate([ext[idx], ext])
    et2 = np.concatenate([et[idx], et]).astype(np.int32)
    nl2 = np.where(nl[idx] >= 0, nl[idx] + K, -1).astype(np.int32)
    return O.eval_ext(K, ext2, et2, nl2)


def sample_centres(n, K=512):
    """The first and the last K centres: the top of the index range exercises
    the largest offsets into the per-slot buffers."""
    return np.concatenate([np.arange(K), np.arange(n - K, n)])


def check_assembly(dp, O, pot, ext, nl, mp, f, v, av, label):
    """Every atom's force, atom virial and the virial of one evaluation
    against the oracle's ProdForce / ProdVirial (orc_prod_force) and ghost
    fold (orc_fold) applied to all of the GPU's per-slot edge gradients, and
    the GPU's mapping against the oracle's. The edge gradients themselves are
    pinned against the oracle on the sampled centres."""
    n = len(nl)
    gmp = pot.stage(dp.STAGE_MAPPING, np.int32, mp.shape)
    assert np.array_equal(gmp, mp), "ghost mapping differs"
    eg = pot.stage(dp.STAGE_EDGE_GRAD, np.float64, (n, O.nnei, 3))
    fr, vr, avr = O.prod_force(n, ext, nl, eg, mapping=mp)
    df, dv, dav = (float(np.abs(a - b).max()) for a, b in ((f, fr), (v, vr), (av, avr)))
    print(f"{label}: assembly from edge gradients: max |dF| {df:.2e}, |dW| {dv:.2e}, "
          f"|d atom_W| {dav:.2e}", flush=True)
    assert df <= F_TOL and dv <= V_TOL and dav <= V_TOL
    return eg


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_full_size_sample_and_invariants(dp, orc, cfg):
    """Atom energies and edge gradients (the backward's output, per slot) of
    1,024 centres against the oracle; every atom's force and atom virial
    against the oracle's assembly of all edge gradients; the size-independent
    properties."""
    O, pot, (coord, atype, box), (e, f, v, ae, av), (ext, et, mp, nl) = _full(dp, orc, cfg)
    n = len(atype)
    idx = sample_centres(n)
    ref = _sample(O, ext, et, nl, idx)
    assert np.abs(ae[idx] - ref["atom_energy"]).max() <= E_TOL
    eg = check_assembly(dp, O, pot, ext, nl, mp, f, v, av, f"config {cfg}")[idx]
    assert np.abs(eg - ref["edge_grad"]).max() <= 1e-11
    assert np.abs(f.sum(0)).max() <= 1e-12 * n
    W = v.reshape(3, 3)
    assert np.abs(W - W.T).max() <= 1e-9 * max(1.0, np.abs(W).max())
    assert np.abs(av.sum(0) - v).max() <= 1e-9 * max(1.0, np.abs(v).max())
    assert abs(e - ae.sum()) <= 1e-9 * max(1.0, abs(e))
