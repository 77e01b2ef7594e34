"""The independent restatement of se_e2_a in torch fp64 (oracle/torch_se_e2_a.py:
batched products, autograd for forces and virial), written from the model's
definition, against the C oracle. It pins the embedding / fitting nets, the
descriptor and the C oracle's hand-written backward, which nothing else pins,
and the torch restatement that bench.py times as its BLAS-backed CPU figure."""
import numpy as np
import pytest

from cases import CASES, FALLBACK_SHAPES, fallback_case, model_bytes

torch = pytest.importorskip("torch")


def torch_eval(m, ext, et, nl, nloc):
    import os
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    from oracle.torch_se_e2_a import torch_eval as te
    return te(m, ext, et, nl, nloc)


@pytest.mark.parametrize("case", ["water192", "hea1024", "cu864"])
def test_torch_matches_oracle(dp, orc, case):
    (coord, atype, box), m = CASES[case]()
    O = orc.Oracle(model_bytes(m))
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    nloc = len(atype)
    ref = O.eval_ext(nloc, ext, et, nl)
    e, f_ext = torch_eval(m, ext, et, nl, nloc)
    np.testing.assert_allclose(ref["atom_energy"], e, rtol=0, atol=1e-12)
    np.testing.assert_allclose(ref["force"], f_ext, rtol=0, atol=1e-11)
    # virial from the autograd forces on the extended system: W = sum x (x) F
    W = (ext[:, :, None] * f_ext[:, None, :]).sum(0)
    np.testing.assert_allclose(ref["virial"].reshape(3, 3), W.T, rtol=0, atol=1e-9)


@pytest.mark.parametrize("name", ["water_axis8_f192", "water_f160"])
def test_torch_matches_oracle_other_fitting_shapes(dp, orc, name):
    """The oracle's descriptor and fitting for axis != 16 and a first fitting
    layer other than 240 wide (the shapes of the GPU fallback-path tests)."""
    assert name in FALLBACK_SHAPES
    (coord, atype, box), m = fallback_case(name)
    O = orc.Oracle(model_bytes(m))
    ext, et, mp, nl = O.neighbor_list(coord, atype, box)
    nloc = len(atype)
    ref = O.eval_ext(nloc, ext, et, nl)
    e, f_ext = torch_eval(m, ext, et, nl, nloc)
    np.testing.assert_allclose(ref["atom_energy"], e, rtol=0, atol=1e-12)
    np.testing.assert_allclose(ref["force"], f_ext, rtol=0, atol=1e-11)
