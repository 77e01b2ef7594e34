"""Pins of the DPA4C-Nano CPU oracle (no GPU): closed forms of every readout
block, the envelope's and the radial table's analytic properties, the
harmonic / STF identities, invariances of the descriptor and finite
differences of the energy. None of these retypes the oracle's vectorised
formulas: the closed forms are derived for one edge with identity readout
matrices, where each invariant reduces to a scalar expression."""
import math

import numpy as np
import pytest
import torch

from _pkg import load_dpa4c_oracle

C4 = load_dpa4c_oracle()


def nano(dp, kind="cu", seed=5, **kw):
    m = dp.dpa4c.random_model(kind, seed=seed, **kw)
    return m, C4.Dpa4cOracle(dp.dpa4c.to_bytes(m))


def test_model_roundtrip_and_independent_reader(dp):
    m = dp.dpa4c.random_model("hea", seed=9)
    buf = dp.dpa4c.to_bytes(m)
    m2 = dp.dpa4c.from_bytes(buf)
    assert dp.dpa4c.to_bytes(m2) == buf
    r = C4.read_model_bytes(buf)
    assert r["ntypes"] == 4 and r["n_int"] == m["interval_count"]
    np.testing.assert_array_equal(r["table"], m["table"].astype(np.float64))
    np.testing.assert_array_equal(r["Pt"], m["Pt"].astype(np.float64))
    np.testing.assert_array_equal(r["layers"][0][0], m["layers"][0][0].astype(np.float64))
    assert r["b_head"] == float(m["b_head"])
    np.testing.assert_array_equal(r["bias"], m["bias_atom_e"])


def test_envelope_closed_form():
    """c3 = (1-x)^4 times the first five Taylor terms of (1-x)^-4, x = r/rc:
    1 - env = 56 x^5 + O(x^6) at 0 and env = 70 (1-x)^4 + O((1-x)^5) at rc."""
    rc = 6.0
    env = lambda r: C4.envelope(torch.tensor([r], dtype=torch.float64), rc).item()  # noqa: E731
    assert env(0.0) == 1.0 and env(rc) == 0.0 and env(rc + 1.0) == 0.0
    for x in (1e-2, 3e-3):
        assert (1.0 - env(x * rc)) / x**5 == pytest.approx(56.0, rel=10 * x)
        assert env(rc * (1.0 - x)) / x**4 == pytest.approx(70.0, rel=10 * x)
    r = torch.linspace(0.05, rc - 0.05, 200, dtype=torch.float64)
    assert torch.all(torch.diff(C4.envelope(r, rc)) < 0)


def test_radial_table_is_c2_across_knots(dp):
    m, O = nano(dp)
    h = m["table_stride"]
    for k in (3, 57, 151, 299):
        rr = torch.tensor([k * h - 1e-9, k * h + 1e-9], dtype=torch.float64, requires_grad=True)
        f = O.radial(rr)
        d1 = torch.stack([torch.autograd.grad(f[:, c].sum(), rr, create_graph=True)[0]
                          for c in range(8)], 1)
        d2 = torch.stack([torch.autograd.grad(d1[:, c].sum(), rr, retain_graph=True)[0]
                          for c in range(8)], 1)
        # fp32 coefficients: continuity to their rounding
        np.testing.assert_allclose(f[0].detach(), f[1].detach(), atol=2e-6)
        np.testing.assert_allclose(d1[0].detach(), d1[1].detach(), atol=2e-4)
        np.testing.assert_allclose(d2[0].detach(), d2[1].detach(), atol=5e-2)


def test_harmonics_and_stf_identity():
    g = torch.Generator().manual_seed(3)
    u = torch.randn(50, 3, generator=g, dtype=torch.float64)
    u = u / u.norm(dim=1, keepdim=True)
    Y = C4.harmonics2(u)
    np.testing.assert_allclose(Y.norm(dim=1), 1.0, atol=1e-14)
    S = C4.stf(Y)
    want = math.sqrt(1.5) * (u[:, :, None] * u[:, None, :] - torch.eye(3, dtype=torch.float64) / 3)
    np.testing.assert_allclose(S, want, atol=1e-14)


def _identity_readout(m):
    m = dict(m)
    m["Ma"] = np.eye(4, dtype=np.float32)
    m["Mt"] = np.eye(4, dtype=np.float32)
    m["Pv"] = np.eye(4, dtype=np.float32)
    m["Pt"] = np.eye(4, dtype=np.float32)[:, :2].copy()
    m["out_mean"] = np.zeros(70, np.float32)
    m["out_inv_std"] = np.ones(70, np.float32)
    return m


def test_single_edge_closed_forms(dp):
    """One centre with one neighbour, eps = 0, identity readout matrices: the
    70 entries in closed form. With a = angular amplitude * angular norm per
    channel, v = a u, STF(t_k) = a_k sqrt(3/2)(uu^T - I/3):
      Gram_rc = a_r a_c (sqrt2 off the diagonal), Bis112 = -2/(3 sqrt5)
      sqrt(3/2) a_f a_s a_k, Bis222 = kappa (3/2)^(3/2) (2/9) a_a a_b a_c,
      Quartic = (2/3) a_t^2 a_v^2, divisors sqrt(mass + floor)."""
    m0 = dp.dpa4c.random_model("hea", seed=21, eps=0.0)
    m = _identity_readout(m0)
    O = C4.Dpa4cOracle(dp.dpa4c.to_bytes(m))
    d = np.array([[1.1, -2.3, 1.7]])
    ti, tj = 2, 1
    atype = np.array([ti, tj])
    D = O.descriptor(torch.tensor(d), torch.tensor([1]), torch.tensor([0]), torch.tensor(atype), 1)
    D = D[0].detach().numpy()
    r = float(np.linalg.norm(d))
    x = r / m["rcut"]
    env = (1 - x) ** 4 * (1 + 4 * x + 10 * x**2 + 20 * x**3 + 35 * x**4)
    i = min(int(r // m["table_stride"]), m["interval_count"] - 1)
    xl = r - i * m["table_stride"]
    coef = m["table"][i].astype(np.float64)
    rad = sum(coef[k] * xl**k for k in range(6))
    film = m["film"][ti * 4 + tj].astype(np.float64)
    amp = (film[:, 0] * rad + film[:, 1]) * env
    fl = m["degree_floor"]
    ns, na = (env**2 + fl) ** -0.5, (env**4 + fl) ** -0.5
    a = amp * env * na
    want = list(amp * ns)
    s2 = math.sqrt(2.0)
    want += [a[p] * a[q] * (1 if p == q else s2) for p in range(4) for q in range(p, 4)]
    want += [a[p] * a[q] * (1 if p == q else s2) for p in range(4) for q in range(p, 4)]
    c112 = -2.0 / (3.0 * math.sqrt(5.0)) * math.sqrt(1.5)
    pairs = [(p, q) for p in range(4) for q in range(p, 4)]
    for o in range(20):
        k = o % 2
        p, q = pairs[o // 2]
        want.append(c112 * a[p] * a[q] * a[k] * (1 if p == q else s2))
    c222 = C4.KAPPA_222 * 1.5**1.5 * 2.0 / 9.0
    for (x1, x2, x3), w in zip(((0, 0, 0), (0, 0, 1), (0, 1, 1), (1, 1, 1)),
                               (1, math.sqrt(3), math.sqrt(3), 1)):
        want.append(c222 * w * a[x1] * a[x2] * a[x3])
    for o in range(8):
        vi, tk = o % 4, o // 4
        want.append(2.0 / 3.0 * a[tk] ** 2 * a[vi] ** 2)
    want += [math.sqrt(env**2 + fl), math.sqrt(env**4 + fl)]
    want += list(m["type_embedding"][ti].astype(np.float64))
    np.testing.assert_allclose(D, np.array(want), rtol=1e-12, atol=1e-14)


def _cluster(seed, n=14, span=4.0):
    rng = np.random.default_rng(seed)
    while True:
        x = rng.uniform(-span, span, (n, 3))
        dd = np.linalg.norm(x[:, None] - x[None], axis=2) + 10 * np.eye(n)
        if dd.min() > 1.2:
            return x


def test_descriptor_invariances(dp):
    """eps = 0: with eps > 0 the direction u = d / sqrt(|d|^2 + eps^2) is
    short of unit length by eps^2 / 2r^2 and the degree-two harmonics (which
    use |u| = 1) are rotation invariant only to that order."""
    m, O = nano(dp, "hea", seed=31, eps=0.0)
    x = _cluster(4)
    atype = np.arange(len(x)) % 4
    base = O.compute(x, atype, None, want_internals=True)
    D0 = base["descriptor"]
    rng = np.random.default_rng(8)
    q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    rot = O.compute(x @ q.T, atype, None, want_internals=True)
    np.testing.assert_allclose(rot["descriptor"], D0, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(rot["force"], base["force"] @ q.T, atol=1e-10)
    tr = O.compute(x + np.array([3.3, -1.2, 0.4]), atype, None, want_internals=True)
    np.testing.assert_allclose(tr["descriptor"], D0, rtol=1e-12, atol=1e-12)
    perm = rng.permutation(len(x))
    pm = O.compute(x[perm], atype[perm], None, want_internals=True)
    np.testing.assert_allclose(pm["descriptor"], D0[perm], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(pm["atom_energy"], base["atom_energy"][perm], rtol=1e-12)
    # an isolated cluster: zero net force and zero net torque
    assert np.abs(base["force"].sum(0)).max() < 1e-10
    assert np.abs(np.cross(x, base["force"]).sum(0)).max() < 1e-10


def test_forces_and_virial_by_finite_differences(dp):
    """A periodic 32-atom Cu cell (box 7.23 A < 2 rcut, ghosts of several
    images): F = -dE/dx and W = -dE/d(strain) by central differences. The
    stored fp32 table coefficients leave jumps of ~1e-7 at the knots, and a
    homogeneous strain moves hundreds of edges across knots at once, so the
    oracle evaluates the unrounded fp64 spline here (the same model drawn
    from the same stream)."""
    m, O = nano(dp, "cu", seed=41)
    tab64, _ = dp.dpa4c.radial_table(dp.systems.Stream(41, 11), m["rcut"], m["table_stride"], 8,
                                     dtype=np.float64)
    np.testing.assert_allclose(tab64, m["table"], rtol=1e-6, atol=1e-6)
    O.T["table"] = torch.as_tensor(tab64)
    coord, atype, box = dp.systems.fcc(2, 3.615, seed=5, sigma=0.1)
    out = O.compute(coord, atype, box)
    E = lambda c, b=box: O.compute(c, atype, b)["energy"]  # noqa: E731
    h = 1e-5
    for a in (0, 7, 19):
        for c in range(3):
            cp, cm = coord.copy(), coord.copy()
            cp[a, c] += h
            cm[a, c] -= h
            fd = -(E(cp) - E(cm)) / (2 * h)
            assert out["force"][a, c] == pytest.approx(fd, abs=2e-8)
    H = box.reshape(3, 3)
    for (p, q) in ((0, 0), (1, 2), (0, 1)):  # upper strains keep h lower-triangular
        eps = np.zeros((3, 3))
        eps[p, q] = h
        Ep = E(coord @ (np.eye(3) + eps).T, (H @ (np.eye(3) + eps).T).ravel())
        Em = E(coord @ (np.eye(3) - eps).T, (H @ (np.eye(3) - eps).T).ravel())
        fd = -(Ep - Em) / (2 * h)
        assert out["virial"][3 * p + q] == pytest.approx(fd, abs=2e-8)
    np.testing.assert_allclose(out["virial"], out["atom_virial"].sum(0), atol=1e-12)
    # symmetric up to the eps^2/r^2 departure from rotation invariance
    W = out["virial"].reshape(3, 3)
    np.testing.assert_allclose(W, W.T, atol=1e-6)
    assert np.abs(out["force"].sum(0)).max() < 1e-10


def test_strict_cutoff(dp):
    """A neighbour at exactly rcut is excluded (r^2 < rcut^2), one just inside
    is kept."""
    m, O = nano(dp, "cu", seed=2)
    rc = m["rcut"]
    for dx, n_edges in ((rc, 0), (np.nextafter(rc, 0.0), 2)):
        x = np.array([[0.0, 0.0, 0.0], [dx, 0.0, 0.0]])
        out = O.compute(x, np.array([0, 0]), None)
        assert len(out["src"]) == n_edges


def test_gaunt_normalisations():
    """The coupling constants are the unit-Frobenius normalisations of the
    Cartesian Gaunt tensors in the packed STF basis (graph_compress.cuh:34-38):
    with S_a = STF(e_a), sum_a |S_a|_F^2 = 5, so the 112 coupling is 1/sqrt5 in
    magnitude, and sum_abc tr(S_a S_b S_c)^2 = 35/12, so the 222 coupling is
    sqrt(12/35) in magnitude. (Their signs are the reference's convention.)"""
    E = torch.eye(5, dtype=torch.float64)
    S = C4.stf(E)                                  # [5, 3, 3]
    np.testing.assert_allclose((S * S).sum(), 5.0, rtol=1e-15)
    t3 = torch.einsum("aij,bjk,cki->abc", S, S, S)
    np.testing.assert_allclose((t3 * t3).sum(), 35.0 / 12.0, rtol=1e-14)
    assert abs(abs(C4.KAPPA_222) - math.sqrt(12.0 / 35.0)) < 1e-15
    # the packed basis is orthonormal under the Frobenius product
    gram = torch.einsum("aij,bij->ab", S, S)
    np.testing.assert_allclose(gram, torch.eye(5, dtype=torch.float64), atol=1e-15)
