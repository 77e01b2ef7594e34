"""Asynchronous device-resident evaluation (dp_compute_device_async, dp_sync):
steps queued back to back with no host round trip give bit-for-bit the
results of the synchronous device entry point, and a capacity error raised by
a queued step is reported by dp_sync instead of being lost."""
import importlib

import numpy as np
import pytest

from cases import CASES, model_bytes

pytestmark = pytest.mark.gpu


def _outputs(hip, n):
    return [hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72),
            hip.DeviceArray(nbytes=8 * n), hip.DeviceArray(nbytes=72 * n)]


def _host(out, n):
    e, f, v, ae, av = out
    return (e.to_host(np.float64, (1,)), f.to_host(np.float64, (n, 3)),
            v.to_host(np.float64, (9,)), ae.to_host(np.float64, (n,)),
            av.to_host(np.float64, (n, 9)))


@pytest.mark.parametrize("case", ["hea1024", "water24_smallbox"])
def test_async_steps_match_sync(dp, case):
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), m = CASES[case]()
    n = len(atype)
    mb = model_bytes(m)
    pot_a = dp.DeepPot(file_content=mb)
    pot_s = dp.DeepPot(file_content=mb)
    rng = np.random.default_rng(17)
    steps = 6
    coords = [coord + rng.normal(0.0, 0.02, coord.shape) for _ in range(steps)]
    da = hip.DeviceArray(atype.astype(np.int32))
    dcs = [hip.DeviceArray(np.ascontiguousarray(c, np.float64)) for c in coords]
    outs = [_outputs(hip, n) for _ in range(steps)]
    for k in range(steps):
        pot_a.compute_device_async(dcs[k].ptr, da.ptr, n, box, *[b.ptr for b in outs[k]],
                                   ago=0 if k == 0 else 1)
    pot_a.sync()
    for k in range(steps):
        ref = _outputs(hip, n)
        pot_s.compute_device(dcs[k].ptr, da.ptr, n, box, *[b.ptr for b in ref], ago=0)
        for got, want in zip(_host(outs[k], n), _host(ref, n)):
            assert np.array_equal(got, want)


def test_async_steps_with_changing_box(dp, orc):
    """NPT-shaped queue: every queued step brings its own cell (isotropic
    scaling, then a tilt), passed by value while earlier steps are still in
    flight. Each step equals the synchronous evaluation on its own cell bit
    for bit, and the last one the oracle at the fp64 bars."""
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), m = CASES["hea1024"]()
    n = len(atype)
    mb = model_bytes(m)
    pot_a = dp.DeepPot(file_content=mb)
    pot_s = dp.DeepPot(file_content=mb)
    H0 = box.reshape(3, 3)
    frac = coord @ np.linalg.inv(H0)
    steps = 5
    boxes, coords = [], []
    for k in range(steps):
        H = H0 * (1.0 + 0.003 * k)
        if k >= 3:
            H[1, 0], H[2, 0], H[2, 1] = 0.02 * k * H0[0, 0], -0.01 * k * H0[0, 0], 0.015 * k * H0[0, 0]
        boxes.append(H.reshape(9).copy())
        coords.append(np.ascontiguousarray(frac @ H, np.float64))
    da = hip.DeviceArray(atype.astype(np.int32))
    dcs = [hip.DeviceArray(c) for c in coords]
    outs = [_outputs(hip, n) for _ in range(steps)]
    hbox = np.zeros(9)
    for k in range(steps):
        hbox[:] = boxes[k]  # one host buffer, rewritten before the queue drains
        pot_a.compute_device_async(dcs[k].ptr, da.ptr, n, hbox, *[b.ptr for b in outs[k]], ago=0)
    pot_a.sync()
    for k in range(steps):
        ref = _outputs(hip, n)
        pot_s.compute_device(dcs[k].ptr, da.ptr, n, boxes[k], *[b.ptr for b in ref], ago=0)
        for got, want in zip(_host(outs[k], n), _host(ref, n)):
            assert np.array_equal(got, want)
    e, f, v, ae, av = _host(outs[-1], n)
    r = orc.Oracle(mb).compute(coords[-1], atype, boxes[-1])
    assert abs(e[0] - r["energy"]) / n <= 1e-10
    assert np.abs(f - r["force"]).max() <= 1e-8
    assert np.abs(v - r["virial"]).max() <= 1e-8


def test_async_capacity_error_reported_by_sync(dp):
    """A perfect FCC lattice at a = 2.2 A puts ~800 atoms within the Cu
    model's 8 A cutoff, above the 512 candidates a centre can hold: the
    neighbour kernel clamps (every access stays in bounds) and raises the
    capacity flag, which the synchronous call reports at once and the
    asynchronous one at dp_sync. The handle then works normally again."""
    hip = importlib.import_module("dpamd.hip")
    coord, atype, box = dp.systems.fcc(4, 2.2, seed=3, sigma=0.0)
    n = len(atype)
    m = dp.model.random_model("cu", seed=1002)
    pot = dp.DeepPot(file_content=model_bytes(m))
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(atype.astype(np.int32))
    out = _outputs(hip, n)
    with pytest.raises(dp.DeepmdException, match="neighbours within rcut"):
        pot.compute_device(dc.ptr, da.ptr, n, box, *[b.ptr for b in out], ago=0)
    pot.compute_device_async(dc.ptr, da.ptr, n, box, *[b.ptr for b in out], ago=0)
    with pytest.raises(dp.DeepmdException, match="neighbours within rcut"):
        pot.sync()
    pot.sync()  # the flag was cleared
    # a normal system on the same handle, queued then synchronised
    (coord2, atype2, box2), _ = CASES["cu864"]()
    n2 = len(atype2)
    dc2 = hip.DeviceArray(np.ascontiguousarray(coord2, np.float64))
    da2 = hip.DeviceArray(atype2.astype(np.int32))
    out2, ref2 = _outputs(hip, n2), _outputs(hip, n2)
    pot.compute_device_async(dc2.ptr, da2.ptr, n2, box2, *[b.ptr for b in out2], ago=0)
    pot.sync()
    pot.compute_device(dc2.ptr, da2.ptr, n2, box2, *[b.ptr for b in ref2], ago=0)
    for got, want in zip(_host(out2, n2), _host(ref2, n2)):
        assert np.array_equal(got, want)


@pytest.mark.parametrize("case", ["hea1024", "cu864"])
def test_graph_replay_matches_eager(dp, monkeypatch, case):
    """DPAMD_GRAPH=1: the third queued call with one key is captured and
    replayed, later ones replay; between replays the coordinates change in
    place and a second handle evaluates them eagerly, and every replay must
    equal that eager result bit for bit (hea1024 forks the per-type fitting
    chains onto their own streams inside the graph, cu864 has one type)."""
    hip = importlib.import_module("dpamd.hip")
    (coord, atype, box), m = CASES[case]()
    n = len(atype)
    mb = model_bytes(m)
    monkeypatch.setenv("DPAMD_GRAPH", "1")
    pot_g = dp.DeepPot(file_content=mb)
    monkeypatch.delenv("DPAMD_GRAPH")
    pot_e = dp.DeepPot(file_content=mb)
    rng = np.random.default_rng(23)
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(atype.astype(np.int32))
    out, ref = _outputs(hip, n), _outputs(hip, n)
    steps = 6
    for k in range(steps):
        dc.upload(np.ascontiguousarray(coord + rng.normal(0.0, 0.02, coord.shape), np.float64))
        pot_g.compute_device_async(dc.ptr, da.ptr, n, box, *[b.ptr for b in out],
                                   ago=0 if k == 0 else 1)
        pot_g.sync()
        pot_e.compute_device(dc.ptr, da.ptr, n, box, *[b.ptr for b in ref], ago=0)
        for got, want in zip(_host(out, n), _host(ref, n)):
            assert np.array_equal(got, want), f"step {k}"
    on, captures, replays = pot_g.graph_stats()
    assert on and captures == 1 and replays == steps - 2, (on, captures, replays)
