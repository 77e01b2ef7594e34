"""Pins of the CPU oracle (no GPU): what fixes each function besides its own
formula — closed forms, brute force, finite differences, invariances, and an
independent torch fp64 autograd restatement (test_torch_crosscheck.py)."""
import numpy as np
import pytest

from cases import CASES, model_bytes


@pytest.fixture(scope="module")
def water(dp, orc):
    (coord, atype, box), m = CASES["water192"]()
    O = orc.Oracle(model_bytes(m))
    return O, coord, atype, box


# ---- switching function -------------------------------------------------
def test_switch_closed_forms(dp, orc):
    O = orc.Oracle(model_bytes(dp.model.random_model("cu", seed=1)))
    rs, rc = O.m["rcut_smth"], O.m["rcut"]
    assert O.switch(rs - 1e-9) == (1.0, 0.0)
    assert O.switch(0.5 * rs) == (1.0, 0.0)
    assert O.switch(rc) == (0.0, 0.0)
    assert O.switch(rc + 1.0) == (0.0, 0.0)
    # smoothstep symmetry: sw(mid) = 1/2 and sw(mid + t) + sw(mid - t) = 1
    mid = 0.5 * (rs + rc)
    assert O.switch(mid)[0] == pytest.approx(0.5, abs=1e-15)
    for t in np.linspace(0.01, 0.49, 9) * (rc - rs):
        assert O.switch(mid + t)[0] + O.switch(mid - t)[0] == pytest.approx(1.0, abs=1e-14)
    # derivative against central differences, and C1/C2 at both ends
    h = 1e-6
    for r in np.linspace(rs + 0.01, rc - 0.01, 25):
        fd = (O.switch(r + h)[0] - O.switch(r - h)[0]) / (2 * h)
        assert O.switch(r)[1] == pytest.approx(fd, abs=1e-8)
    for edge in (rs, rc):
        d_in = O.switch(edge - 1e-7 if edge == rc else edge + 1e-7)[1]
        assert abs(d_in) < 1e-9
    # second derivative vanishes at the ends: dsw changes like (r-rs)^2
    e = 1e-3
    assert abs(O.switch(rs + e)[1]) < 40.0 * e * e / (rc - rs) ** 3 * (rc - rs)


def test_env_mat_single_neighbour(dp, orc):
    """Two atoms in an open system: the env row is the closed form and its
    derivative the central difference."""
    m = dp.model.random_model("water", seed=3)
    O = orc.Oracle(model_bytes(m))
    d = np.array([1.3, -0.7, 2.1])
    ext = np.array([[0.0, 0.0, 0.0], d])
    et = np.array([0, 1], np.int32)
    nl = np.full((1, O.nnei), -1, np.int32)
    nl[0, O.sec[1]] = 1
    env, envd, rij = O.env_mat(1, ext, et, nl)
    r = np.linalg.norm(d)
    sw, dsw = O.switch(r)
    avg = m["davg"][0, 1]
    std = m["dstd"][0, 1]
    raw = np.array([sw / r, sw * d[0] / r**2, sw * d[1] / r**2, sw * d[2] / r**2])
    np.testing.assert_allclose(env[0, O.sec[1]], (raw - avg) / std, rtol=1e-14, atol=1e-14)
    np.testing.assert_allclose(rij[0, O.sec[1]], d, rtol=0, atol=0)
    # padded slot of section 0: (0 - avg)/std, derivative 0
    np.testing.assert_allclose(env[0, 0], (0.0 - m["davg"][0, 0]) / m["dstd"][0, 0], rtol=1e-15)
    assert np.all(envd[0, 0] == 0.0)
    h = 1e-6
    for c in range(3):
        ep = ext.copy(); ep[1, c] += h
        em = ext.copy(); em[1, c] -= h
        fd = (O.env_mat(1, ep, et, nl)[0] - O.env_mat(1, em, et, nl)[0])[0, O.sec[1]] / (2 * h)
        np.testing.assert_allclose(envd[0, O.sec[1], :, c], fd, rtol=1e-6, atol=1e-8)


# ---- neighbour lists ------------------------------------------------------
@pytest.mark.parametrize("case", list(CASES))
def test_candidates_brute_equals_cell(orc, case):
    (coord, atype, box), m = CASES[case]()
    O = orc.Oracle(model_bytes(m))
    ext, et, mp = O.ghosts(coord, atype, box, O.m["rcut"])
    nloc = len(atype)
    ob, cb = O.candidates(nloc, ext, et, O.m["rcut"], "brute")
    oc, cc = O.candidates(nloc, ext, et, O.m["rcut"], "cell")
    assert np.array_equal(ob, oc) and np.array_equal(cb, cc)


def test_ghosts_cover_every_image_within_rcut(orc, dp):
    """Every periodic image within rcut of a local atom is present exactly once."""
    (coord, atype, box), m = CASES["water24_smallbox"]()
    O = orc.Oracle(model_bytes(m))
    rc = O.m["rcut"]
    ext, et, mp = O.ghosts(coord, atype, box, rc)
    nloc = len(atype)
    assert np.array_equal(mp[:nloc], np.arange(nloc))
    L = box[0]
    wrapped = ext[:nloc]
    for i in range(nloc):
        # brute force over images of every atom
        cnt = 0
        for k in range(nloc):
            for sh in np.stack(np.meshgrid(*[np.arange(-2, 3)] * 3, indexing="ij"), -1).reshape(-1, 3):
                if k == i and not sh.any():
                    continue
                if np.sum((wrapped[k] + L * sh - wrapped[i]) ** 2) <= rc * rc:
                    cnt += 1
        d2 = np.sum((ext - ext[i]) ** 2, axis=1)
        d2[i] = np.inf
        assert (d2 <= rc * rc).sum() == cnt
    # each ghost is its owner shifted by an integer lattice vector
    shift = (ext - ext[mp]) / L
    assert np.abs(shift - np.rint(shift)).max() < 1e-12


def test_ghosts_cover_every_image_triclinic(orc, dp):
    """Triclinic cell smaller than 2 rcut: every image x_k + n_a a + n_b b +
    n_c c within rcut of a local atom is present exactly once, and each
    ghost is its owner shifted by an integer combination of the lattice
    vectors (rows of h)."""
    (coord, atype, box), m = CASES["water24_tric"]()
    O = orc.Oracle(model_bytes(m))
    rc = O.m["rcut"]
    H = box.reshape(3, 3)
    ext, et, mp = O.ghosts(coord, atype, box, rc)
    nloc = len(atype)
    assert np.array_equal(mp[:nloc], np.arange(nloc))
    wrapped = ext[:nloc]
    shifts = np.stack(np.meshgrid(*[np.arange(-4, 5)] * 3, indexing="ij"), -1).reshape(-1, 3)
    lat = shifts @ H
    for i in range(nloc):
        cnt = 0
        for k in range(nloc):
            d2 = np.sum((wrapped[k] + lat - wrapped[i]) ** 2, axis=1)
            if k == i:
                d2[np.all(shifts == 0, axis=1)] = np.inf
            cnt += int((d2 <= rc * rc).sum())
        d2 = np.sum((ext - ext[i]) ** 2, axis=1)
        d2[i] = np.inf
        assert (d2 <= rc * rc).sum() == cnt
    # the image shifts reach past the searched range only if the brute force
    # above could have missed images: the largest shift used must be inside it
    n = (ext - ext[mp]) @ np.linalg.inv(H)
    assert np.abs(n - np.rint(n)).max() < 1e-9
    assert np.abs(np.rint(n)).max() < 4


def _nlist_of(O, ext, et):
    nloc = 1
    off = np.array([0, len(et) - 1], np.int64)
    cand = np.arange(1, len(et), dtype=np.int32)
    return O.format_nlist(nloc, ext, et, off, cand)[0]


def test_format_nlist_rules(dp, orc):
    m = dp.model.random_model("water", seed=5, sel=[3, 2])
    O = orc.Oracle(model_bytes(m))
    rc = O.m["rcut"]
    # centre 0 (type 0); candidates 1..: type, position
    pts = [(0, [0, 0, 0]),
           (1, [1.0, 0, 0]),     # j=1, H r=1
           (0, [0, 2.0, 0]),     # j=2, O r=2
           (0, [0, 0, 2.0]),     # j=3, O r=2 (tie with j=2 -> j order)
           (1, [0, 0.5, 0]),     # j=4, H r=0.5
           (0, [rc, 0, 0]),      # j=5, O at exactly rcut: kept (r2 <= rc^2)
           (0, [0, rc + 1e-9, 0]),  # j=6, just outside
           (1, [3.0, 0, 0]),     # j=7, H r=3 -> third H, dropped (sel 2)
           (0, [1.5, 0, 0]),     # j=8, O r=1.5
           ]
    ext = np.array([p for _, p in pts], float)
    et = np.array([t for t, _ in pts], np.int32)
    row = _nlist_of(O, ext, et)
    # O section (sel 3): r=1.5 (j8), r=2 (j2), r=2 (j3); j5 at rcut is 4th -> dropped
    assert list(row[:3]) == [8, 2, 3]
    # H section (sel 2): r=0.5 (j4), r=1 (j1); j7 dropped
    assert list(row[3:5]) == [4, 1]
    # with a larger O sel the rcut atom is kept and padding follows
    m2 = dp.model.random_model("water", seed=5, sel=[6, 4])
    O2 = orc.Oracle(model_bytes(m2))
    row2 = _nlist_of(O2, ext, et)
    assert list(row2[:6]) == [8, 2, 3, 5, -1, -1]
    assert list(row2[6:]) == [4, 1, 7, -1]


def test_nlist_sorted_and_within_cutoff(water, orc):
    O, coord, atype, box = water
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    rc2 = O.m["rcut"] ** 2
    for i in range(len(atype)):
        for t in range(2):
            sec = nl[i, O.sec[t]:O.sec[t + 1]]
            real = sec[sec >= 0]
            assert np.all(sec[len(real):] == -1)
            assert np.all(et[real] == t)
            d2 = np.sum((ext[real] - ext[i]) ** 2, axis=1)
            assert np.all(d2 <= rc2)
            keys = list(zip(d2, real))
            assert keys == sorted(keys)


# ---- energy, force, virial -------------------------------------------------
@pytest.mark.parametrize("case", ["water192", "hea1024", "water24_tric"])
def test_force_is_minus_gradient(orc, case):
    (coord, atype, box), m = CASES[case]()
    O = orc.Oracle(model_bytes(m))
    out = O.compute(coord, atype, box)
    h = 1e-5
    rng = np.random.default_rng(0)
    for a in rng.choice(len(atype), 4, replace=False):
        for c in range(3):
            cp = coord.copy(); cp[a, c] += h
            cm = coord.copy(); cm[a, c] -= h
            fd = -(O.compute(cp, atype, box)["energy"] - O.compute(cm, atype, box)["energy"]) / (2 * h)
            assert out["force"][a, c] == pytest.approx(fd, abs=2e-7)


@pytest.mark.parametrize("case", ["water192", "cu864", "water24_tric"])
def test_virial_is_minus_strain_derivative(orc, case):
    (coord, atype, box), m = CASES[case]()
    O = orc.Oracle(model_bytes(m))
    out = O.compute(coord, atype, box)
    W = out["virial"].reshape(3, 3)
    h = 1e-6
    for a in range(3):
        for b in range(a + 1):
            e = np.zeros((3, 3)); e[a, b] = h
            def en(G):
                return O.compute(coord @ G, atype, (box.reshape(3, 3) @ G).reshape(9))["energy"]
            fd = -(en(np.eye(3) + e) - en(np.eye(3) - e)) / (2 * h)
            assert W[a, b] == pytest.approx(fd, abs=2e-5 * max(1.0, abs(fd)))
    assert np.abs(W - W.T).max() < 1e-10
    np.testing.assert_allclose(out["atom_virial"].sum(0), out["virial"], rtol=0, atol=1e-10)
    assert np.abs(out["force"].sum(0)).max() < 1e-10


def test_atom_virial_split_and_orientation(dp, orc):
    """Per-atom virial pinned element by element, not only through its sum.

    One oxygen centre carries all the energy: the hydrogen fitting net and its
    bias_atom_e are zero, so every hydrogen's atom energy is exactly 0 and so
    are the gradients of the edges it centres. Each edge (0 -> j) then carries
    g_j = dE/d(x_j - x_0) = -F_j, and F_j is taken here by central differences
    of the energy, independently of the oracle's backward. The reference
    charges -g (x) d to the edge's neighbour (source) atom with row = gradient
    component (deepmd-op/overlays/op/pt/edge_force_virial.cu:8-9, :138-146),
    so atom_virial[j][3c + d] = F_j[c] (x_j - x_0)[d] and the centre gets 0.
    Charging the centre, or transposing the 3x3, fails here: the expected
    matrices are far from symmetric because se_e2_a edge gradients are not
    radial."""
    m = dp.model.random_model("water", seed=11)
    m["fit_params"][1, :] = 0.0
    m["bias_atom_e"][1] = 0.0
    O = orc.Oracle(model_bytes(m))
    ext0 = np.array([[0.0, 0.0, 0.0],
                     [0.93, 0.31, -0.22],
                     [-0.41, 1.17, 0.35],
                     [2.10, -1.30, 1.90],
                     [-1.70, -2.40, -0.80],
                     [0.60, 3.10, -2.70]])
    et = np.array([0, 1, 1, 1, 1, 1], np.int32)
    n = len(et)

    def run(ext):
        off, cand = O.candidates(n, ext, et, O.m["rcut"], "brute")
        return O.eval_ext(n, ext, et, O.format_nlist(n, ext, et, off, cand))

    out = run(ext0)
    assert np.all(out["atom_energy"][1:] == 0.0)
    av = out["atom_virial"].reshape(n, 3, 3)
    assert np.all(av[0] == 0.0)
    h = 1e-5
    asym = 0.0
    for j in range(1, n):
        fj = np.zeros(3)
        for c in range(3):
            ep = ext0.copy(); ep[j, c] += h
            em = ext0.copy(); em[j, c] -= h
            fj[c] = -(run(ep)["energy"] - run(em)["energy"]) / (2 * h)
        np.testing.assert_allclose(out["force"][j], fj, rtol=0, atol=1e-7)
        expect = np.outer(fj, ext0[j] - ext0[0])
        np.testing.assert_allclose(av[j], expect, rtol=0, atol=1e-6)
        asym = max(asym, np.abs(expect - expect.T).max())
    # the transposed split would miss by far more than the tolerance
    assert asym > 100 * 1e-6
    np.testing.assert_allclose(av.sum(0).reshape(9), out["virial"], rtol=0, atol=1e-12)


def test_prod_force_reassembles_eval(orc):
    """orc_prod_force + orc_fold applied to the oracle's own edge gradients
    give the forces / virials / atom virials of compute() bit for bit (the
    GPU full-size tests use this assembly as the per-atom check), and a
    planted routing mistake (two neighbour indices swapped in one row, or the
    ghost mapping shifted by one) changes the result far beyond 1e-8."""
    (coord, atype, box), m = CASES["water192"]()
    O = orc.Oracle(model_bytes(m))
    out = O.compute(coord, atype, box)
    ext, mp, nl, eg = out["ext_coord"], out["mapping"], out["nlist"], out["edge_grad"]
    n = len(atype)
    f, v, av = O.prod_force(n, ext, nl, eg, mapping=mp)
    assert np.array_equal(f, out["force"]) and np.array_equal(v, out["virial"])
    assert np.array_equal(av, out["atom_virial"])
    nl2 = nl.copy()
    nl2[5, [0, 1]] = nl2[5, [1, 0]]
    assert np.abs(O.prod_force(n, ext, nl2, eg, mapping=mp)[0] - f).max() > 1e-4
    mp2 = mp.copy()
    mp2[n:] = (mp2[n:] + 1) % n
    f2, _, av2 = O.prod_force(n, ext, nl, eg, mapping=mp2)
    assert np.abs(f2 - f).max() > 1e-4 and np.abs(av2 - av).max() > 1e-4


def test_invariances(dp, orc, water):
    O, coord, atype, box = water
    e0 = O.compute(coord, atype, box)
    # translation (periodic: rewrapping changes coordinates, not the energy)
    e1 = O.compute(coord + np.array([3.1, -7.7, 40.2]), atype, box)
    assert e1["energy"] == pytest.approx(e0["energy"], abs=1e-10)
    np.testing.assert_allclose(e1["force"], e0["force"], atol=1e-10)
    # permutation of atoms
    perm = np.random.default_rng(1).permutation(len(atype))
    e2 = O.compute(coord[perm], atype[perm], box)
    assert e2["energy"] == pytest.approx(e0["energy"], abs=1e-10)
    np.testing.assert_allclose(e2["force"], e0["force"][perm], atol=1e-10)
    # rotation of an open cluster
    sub = coord[:24]
    ts = atype[:24]
    th = 0.7
    R = np.array([[np.cos(th), -np.sin(th), 0], [np.sin(th), np.cos(th), 0], [0, 0, 1.0]])
    R = R @ np.array([[1, 0, 0], [0, np.cos(0.3), -np.sin(0.3)], [0, np.sin(0.3), np.cos(0.3)]])
    ext = sub.copy()
    off, cand = O.candidates(24, ext, ts, O.m["rcut"], "brute")
    nl = O.format_nlist(24, ext, ts, off, cand)
    a = O.eval_ext(24, ext, ts, nl)
    ext2 = sub @ R.T
    off2, cand2 = O.candidates(24, ext2, ts, O.m["rcut"], "brute")
    b = O.eval_ext(24, ext2, ts, O.format_nlist(24, ext2, ts, off2, cand2))
    assert b["energy"] == pytest.approx(a["energy"], abs=1e-10)
    np.testing.assert_allclose(b["force"], a["force"] @ R.T, atol=1e-10)
    # rotation invariance of an isolated cluster: no net force, no net torque
    assert np.abs(a["force"].sum(0)).max() < 1e-10
    assert np.abs(np.cross(sub, a["force"]).sum(0)).max() < 1e-9


def test_padded_slots_use_net_at_s_pad(dp, orc):
    """An isolated atom has only padded slots: T = R_pad^T G(s_pad) per section."""
    m = dp.model.random_model("water", seed=9)
    O = orc.Oracle(model_bytes(m))
    ext = np.zeros((1, 3))
    et = np.zeros(1, np.int32)
    nl = np.full((1, O.nnei), -1, np.int32)
    out = O.eval_ext(1, ext, et, nl, want_internals=True)
    L3, M2 = m["emb"][2], m["axis"]
    T = np.zeros((4, L3))
    for t in range(2):
        rpad = (0.0 - m["davg"][0, t]) / m["dstd"][0, t]
        T += O.m["sel"][t] * np.outer(rpad, O.embed(0, t, rpad[0]))
    T /= O.nnei
    D = T.T @ T[:, :M2]
    np.testing.assert_allclose(out["descrpt"][0], D.reshape(-1), rtol=1e-13, atol=1e-15)
    assert np.all(out["force"] == 0.0)
