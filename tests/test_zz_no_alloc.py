"""dp_compute_device_noalloc: the device-resident evaluation with every work
buffer carved from the library's static per-GPU scratch. Its outputs are
checked against dp_compute_device's on the same handle to the fp64 bar of the
parity tests (energy per atom <= 1e-10 eV, forces <= 1e-8 eV/A, virials
<= 1e-8 eV), on two calls in a row with the second input smaller, so that the
second call runs over what the first left in the scratch. The handle's own
buffers and the device's free memory are unchanged by the calls, and a system
larger than the scratch is rejected without breaking the handle."""
import ctypes as C
import importlib

import numpy as np
import pytest

from cases import CASES, fallback_case, model_bytes

pytestmark = pytest.mark.gpu

E_TOL = 1e-10   # eV per atom
F_TOL = 1e-8    # eV/A
V_TOL = 1e-8    # eV


def _outputs(hip, n):
    return [hip.DeviceArray(nbytes=8), hip.DeviceArray(nbytes=24 * n), hip.DeviceArray(nbytes=72),
            hip.DeviceArray(nbytes=8 * n), hip.DeviceArray(nbytes=72 * n)]


def _host(out, n):
    e, f, v, ae, av = out
    return (e.to_host(np.float64, (1,))[0], f.to_host(np.float64, (n, 3)),
            v.to_host(np.float64, (9,)), ae.to_host(np.float64, (n,)),
            av.to_host(np.float64, (n, 9)))


def _free_bytes(hip):
    h = hip.hip()
    h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    free, total = C.c_size_t(0), C.c_size_t(0)
    hip.check(h.hipMemGetInfo(C.byref(free), C.byref(total)))
    return free.value


def _both(hip, pot, system):
    """(noalloc outputs, dp_compute_device outputs) on host for one system;
    the no-allocation call goes first, on poisoned output buffers."""
    coord, atype, box = system
    n = len(atype)
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(np.ascontiguousarray(atype, np.int32))
    got, ref = _outputs(hip, n), _outputs(hip, n)
    for b in got:
        b.upload(np.full(b.nbytes // 8, np.nan))
    pot.compute_device_noalloc(dc.ptr, da.ptr, n, box, *[b.ptr for b in got])
    pot.compute_device(dc.ptr, da.ptr, n, box, *[b.ptr for b in ref], ago=0)
    return _host(got, n), _host(ref, n)


def _check(got, ref, n):
    e, f, v, ae, av = got
    e0, f0, v0, ae0, av0 = ref
    assert abs(e - e0) / n <= E_TOL
    assert np.abs(ae - ae0).max() <= E_TOL
    assert np.abs(f - f0).max() <= F_TOL
    assert np.abs(v - v0).max() <= V_TOL
    assert np.abs(av - av0).max() <= V_TOL


@pytest.mark.parametrize("case", ["water192", "hea250", "hea250_mixed", "water_axis8",
                                  "water_axis8_mixed", "dpa4c_hea250"])
def test_noalloc_matches_device_entry_point_twice(dp, case):
    """Two calls in a row on one handle, the second with a smaller system
    (192 water atoms -> 24 in a small box; 250 HEA atoms of four types ->
    128, in fp64 and in mixed precision; the water model with a fitting shape
    outside the fused kernels; a DPA4C-Nano model on the HEA pair), then the
    first again: each agrees with dp_compute_device. The saved fp64 embedding activations (16 (L2P +
    L3P) doubles per 16-slot tile: 295 KB per HEA atom, 221 KB per Cu atom)
    bound what fits in 128 MiB; the mixed path saves none."""
    hip = importlib.import_module("dpamd.hip")
    if case == "water192":
        (coord, atype, box), m = CASES[case]()
        small = CASES["water24_smallbox"]()[0]
    elif case.startswith("water_axis8"):
        # a fitting shape without the fused input-gradient kernels (axis 8,
        # first layer 192 wide): stored D, the plain dE/dD GEMM, any-axis dE/dT
        (coord, atype, box), m = fallback_case("water_axis8_f192")
        small = CASES["water24_smallbox"]()[0]
    elif case == "dpa4c_hea250":
        m = None
        coord, atype, box = dp.systems.bcc_hea(5, 3.2, seed=8)
        small = dp.systems.bcc_hea(4, 3.2, seed=36)
    else:
        m = CASES["hea1024"]()[1]
        coord, atype, box = dp.systems.bcc_hea(5, 3.2, seed=35)
        small = dp.systems.bcc_hea(4, 3.2, seed=36)
    prec = dp.PREC_MIXED if case.endswith("_mixed") else dp.PREC_FP64
    mb = dp.dpa4c.to_bytes(dp.dpa4c.random_model("hea", seed=307)) if m is None else model_bytes(m)
    pot = dp.DeepPot(file_content=mb, precision=prec)
    bytes0 = pot.device_bytes()
    big = (coord, atype, box)
    for system in (big, small, big):
        got, ref = _both(hip, pot, system)
        _check(got, ref, len(system[1]))
    # the handle's own buffers were only sized by dp_compute_device
    pot2 = dp.DeepPot(file_content=mb, precision=prec)
    n = len(atype)
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(np.ascontiguousarray(atype, np.int32))
    out = _outputs(hip, n)
    pot2.compute_device_noalloc(dc.ptr, da.ptr, n, box, *[b.ptr for b in out])
    assert pot2.device_bytes() == bytes0


def test_noalloc_allocates_no_device_memory(dp):
    """After one warm-up call (which loads the kernels' code objects), further
    calls of other sizes leave the device's free memory exactly as it was."""
    hip = importlib.import_module("dpamd.hip")
    m = CASES["cu864"]()[1]
    pot = dp.DeepPot(file_content=model_bytes(m))
    bytes0 = pot.device_bytes()
    systems = [dp.systems.fcc(4, 3.615, seed=4), dp.systems.fcc(3, 3.615, seed=5)]
    bufs = []
    for c, a, b in systems:
        n = len(a)
        bufs.append((hip.DeviceArray(np.ascontiguousarray(c, np.float64)),
                     hip.DeviceArray(np.ascontiguousarray(a, np.int32)), _outputs(hip, n), n, b))
    dc, da, out, n, b = bufs[0]
    pot.compute_device_noalloc(dc.ptr, da.ptr, n, b, *[x.ptr for x in out])
    hip.synchronize()
    free0 = _free_bytes(hip)
    for dc, da, out, n, b in (bufs[1], bufs[0], bufs[1]):
        pot.compute_device_noalloc(dc.ptr, da.ptr, n, b, *[x.ptr for x in out])
    hip.synchronize()
    assert _free_bytes(hip) == free0
    assert pot.device_bytes() == bytes0


def test_noalloc_rejects_system_beyond_scratch(dp):
    """2048 Cu atoms need about 450 MB of saved activations, beyond the
    128 MiB scratch: the call fails with a capacity error naming the limit,
    and both entry points work on the handle afterwards."""
    hip = importlib.import_module("dpamd.hip")
    m = CASES["cu864"]()[1]
    coord, atype, box = dp.systems.fcc(4, 3.615, seed=4)
    pot = dp.DeepPot(file_content=model_bytes(m))
    cb, ab, bb = dp.systems.fcc(8, 3.615, seed=6)
    nb = len(ab)
    dc = hip.DeviceArray(np.ascontiguousarray(cb, np.float64))
    da = hip.DeviceArray(np.ascontiguousarray(ab, np.int32))
    out = _outputs(hip, nb)
    with pytest.raises(dp.DeepmdException, match="MiB of static scratch"):
        pot.compute_device_noalloc(dc.ptr, da.ptr, nb, bb, *[x.ptr for x in out])
    got, ref = _both(hip, pot, (coord, atype, box))
    _check(got, ref, len(atype))


def test_noalloc_refuses_a_capturing_stream(dp):
    """The call reads the atom types back and synchronises, so on a stream
    under graph capture it returns an argument error before touching the
    stream; the capture then ends cleanly (an empty graph) and the handle
    keeps working."""
    hip = importlib.import_module("dpamd.hip")
    h = hip.hip()
    P = C.c_void_p
    h.hipStreamCreate.argtypes = [C.POINTER(P)]
    h.hipStreamDestroy.argtypes = [P]
    h.hipStreamBeginCapture.argtypes = [P, C.c_int]
    h.hipStreamEndCapture.argtypes = [P, C.POINTER(P)]
    h.hipGraphDestroy.argtypes = [P]
    (coord, atype, box), m = CASES["water192"]()
    pot = dp.DeepPot(file_content=model_bytes(m))
    n = len(atype)
    dc = hip.DeviceArray(np.ascontiguousarray(coord, np.float64))
    da = hip.DeviceArray(np.ascontiguousarray(atype, np.int32))
    out = _outputs(hip, n)
    st = P()
    hip.check(h.hipStreamCreate(C.byref(st)))
    try:
        hip.check(h.hipStreamBeginCapture(st, 2))  # hipStreamCaptureModeRelaxed
        with pytest.raises(dp.DeepmdException, match="graph capture"):
            pot.compute_device_noalloc(dc.ptr, da.ptr, n, box, *[b.ptr for b in out],
                                       stream=st.value)
        g = P()
        hip.check(h.hipStreamEndCapture(st, C.byref(g)))
        if g.value:
            hip.check(h.hipGraphDestroy(g))
    finally:
        hip.check(h.hipStreamDestroy(st))
    got, ref = _both(hip, pot, (coord, atype, box))
    _check(got, ref, n)
