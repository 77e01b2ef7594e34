"""The oracle against the committed golden fixtures (tests/golden/)."""
import hashlib
import json
import os

import numpy as np
import pytest

from cases import CASES, model_bytes

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(case):
    with open(os.path.join(HERE, f"{case}.json")) as f:
        doc = json.load(f)
    unhex = lambda v: np.array([float.fromhex(x) for x in v])  # noqa: E731
    return doc, unhex


@pytest.mark.parametrize("case", ["water192", "cu864"])
def test_inputs_unchanged(case):
    doc, _ = load(case)
    (coord, atype, box), m = CASES[case]()
    assert hashlib.sha256(model_bytes(m)).hexdigest() == doc["model_sha256"]
    assert hashlib.sha256(np.ascontiguousarray(coord).tobytes()).hexdigest() == doc["coord_sha256"]


@pytest.mark.parametrize("case", ["water192", "cu864"])
def test_oracle_reproduces_golden(orc, case):
    doc, unhex = load(case)
    (coord, atype, box), m = CASES[case]()
    out = orc.Oracle(model_bytes(m)).compute(coord, atype, box)
    assert len(out["ext_type"]) == doc["nall"]
    assert hashlib.sha256(out["nlist"].astype(np.int32).tobytes()).hexdigest() == doc["nlist_sha256"]
    if case == "water192":
        z = np.load(os.path.join(HERE, "water192.npz"))
        assert np.array_equal(z["nlist"], out["nlist"])
        assert np.array_equal(z["mapping"], out["mapping"])
    assert out["energy"] == pytest.approx(float.fromhex(doc["energy"]), abs=1e-10)
    np.testing.assert_allclose(out["atom_energy"], unhex(doc["atom_energy"]), rtol=0, atol=1e-12)
    np.testing.assert_allclose(out["force"].reshape(-1), unhex(doc["force"]), rtol=0, atol=1e-11)
    np.testing.assert_allclose(out["virial"], unhex(doc["virial"]), rtol=0, atol=1e-10)


def test_cu_sel_overflow_present(orc):
    """The Cu fixture exercises truncation: 176 atoms within 8 A, sel keeps 138."""
    (coord, atype, box), m = CASES["cu864"]()
    O = orc.Oracle(model_bytes(m))
    ext, et, mp = O.ghosts(coord, atype, box, O.m["rcut"])
    off, cand = O.candidates(len(atype), ext, et, O.m["rcut"], "cell")
    counts = np.diff(off)
    assert counts.min() >= 170 and counts.max() <= 190
    nl = O.format_nlist(len(atype), ext, et, off, cand)
    assert np.all(nl >= 0)
