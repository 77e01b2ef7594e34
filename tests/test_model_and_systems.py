"""Model file format and seeded synthetic systems (host logic, no GPU)."""
import numpy as np
import pytest


def test_model_roundtrip_and_independent_reader(dp, orc):
    m = dp.model.random_model("hea", seed=11)
    b = dp.model.to_bytes(m)
    m2 = dp.model.from_bytes(b)
    assert dp.model.to_bytes(m2) == b
    r = orc.read_model_bytes(b)
    assert r["sel"] == m["sel"] and r["emb"] == m["emb"] and r["fit"] == m["fit"]
    np.testing.assert_array_equal(r["emb_params"], m["emb_params"].reshape(-1))
    np.testing.assert_array_equal(r["fit_params"], m["fit_params"].reshape(-1))
    with pytest.raises(ValueError):
        dp.model.from_bytes(b"XXXXXXXX" + b[8:])


def test_model_seeded(dp):
    a = dp.model.to_bytes(dp.model.random_model("cu", seed=3))
    b = dp.model.to_bytes(dp.model.random_model("cu", seed=3))
    c = dp.model.to_bytes(dp.model.random_model("cu", seed=4))
    assert a == b and a != c


def test_prng_known_values(dp):
    # splitmix64 counter stream: first outputs for seed 0, stream 0 are fixed
    s = dp.systems.Stream(0, 0)
    v = s.bits(3)
    s2 = dp.systems.Stream(0, 0)
    assert np.array_equal(v, s2.bits(3))
    u = dp.systems.Stream(1, 2).uniform(100000)
    assert 0.0 <= u.min() and u.max() < 1.0 and abs(u.mean() - 0.5) < 5e-3
    g = dp.systems.Stream(1, 3).normal(200000)
    assert abs(g.mean()) < 1e-2 and abs(g.std() - 1.0) < 1e-2


@pytest.mark.parametrize("cfg,natoms,edge", [(0, 192, 12.42), (1, 12288, 49.68), (2, 131072, 115.68),
                                              (3, 128000, 128.0), (4, 393216, 157.5)])
def test_benchmark_systems(dp, cfg, natoms, edge):
    coord, atype, box = dp.systems.build(cfg)
    assert coord.shape == (natoms, 3) and atype.shape == (natoms,)
    assert box[0] == pytest.approx(edge) and box[4] == pytest.approx(edge) and box[8] == pytest.approx(edge)
    assert box[1] == box[2] == box[3] == box[5] == box[6] == box[7] == 0.0
    if cfg in (0, 1, 4):
        nmol = natoms // 3
        assert np.all(atype[:nmol] == 0) and np.all(atype[nmol:] == 1)
        o = coord[:nmol]
        h = coord[nmol:].reshape(nmol, 2, 3)
        np.testing.assert_allclose(np.linalg.norm(h - o[:, None], axis=2), 0.96, atol=1e-12)
        v1, v2 = h[:, 0] - o, h[:, 1] - o
        ang = np.degrees(np.arccos(np.sum(v1 * v2, 1) / 0.96**2))
        np.testing.assert_allclose(ang, 104.52, atol=1e-9)
    if cfg == 3:
        assert np.array_equal(np.bincount(atype), [32000] * 4)
    if cfg == 2:
        assert np.all(atype == 0)
        a = 3.615
        frac = coord / a * 2
        assert np.abs(frac - np.rint(frac)).max() < 0.2 * 2 / a * 3  # jitter sigma 0.05 A


def test_lammps_list_matches_brute_force(dp):
    """The host-side LAMMPS-style list (ghosts appended after the local atoms,
    all atoms within the cutoff of each local atom): neighbour sets equal a
    brute-force search over the extended atoms, counts equal the minimum
    image's, ghosts are images of local atoms."""
    coord, atype, box = dp.systems.build(1)
    cut = 7.0
    ext, et, nghost, off, nb = dp.systems.lammps_list(coord, atype, box, cut)
    n = len(atype)
    assert len(et) == n + nghost and off[0] == 0 and off[-1] == len(nb)
    L = np.diag(np.asarray(box, np.float64).reshape(3, 3))
    # ghosts are periodic images of local atoms of the same type
    assert nghost > 0
    rng = np.random.default_rng(0)
    for gi in rng.choice(nghost, 20, replace=False):
        dg = coord - ext[n + gi]
        dg -= np.round(dg / L) * L
        k = int(np.argmin(np.einsum("ij,ij->i", dg, dg)))
        assert np.abs(dg[k]).max() < 1e-9 and atype[k] == et[n + gi]
    for i in rng.choice(n, 12, replace=False):
        dd = np.linalg.norm(ext - ext[i], axis=1)
        want = set(np.nonzero(dd < cut)[0].tolist()) - {int(i)}
        assert want == set(nb[off[i]:off[i + 1]].tolist())
        m = coord - coord[i]
        m -= np.round(m / L) * L
        assert int((np.einsum("ij,ij->i", m, m) < cut * cut).sum()) - 1 == off[i + 1] - off[i]
    assert np.all(et[n:] >= 0)
