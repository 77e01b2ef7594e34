"""Independent restatement of se_e2_a in torch fp64 (autograd for forces and
virial), written from the model's definition, against the C oracle. It pins
the embedding/fitting nets, the descriptor and the oracle's hand-written
backward, which nothing else pins."""
import numpy as np
import pytest

from cases import CASES, FALLBACK_SHAPES, fallback_case, model_bytes

torch = pytest.importorskip("torch")


def _net_layers(params, widths_in, widths_out):
    out, p = [], 0
    for i, o in zip(widths_in, widths_out):
        W = params[p:p + i * o].reshape(i, o); p += i * o
        b = params[p:p + o]; p += o
        out.append((W, b))
    return out, p


def _act(x, W, b, idt=None):
    t = torch.tanh(x @ W + b)
    i, o = W.shape
    if o == i:
        return x + (idt * t if idt is not None else t)
    if o == 2 * i:
        return torch.cat([x, x], dim=-1) + t
    return t


def torch_eval(m, ext, et, nl, nloc):
    nt = len(m["type_map"])
    sel = m["sel"]
    sec = np.concatenate([[0], np.cumsum(sel)])
    nnei = int(sec[-1])
    L1, L2, L3 = m["emb"]
    M2 = m["axis"]
    rs, rc = m["rcut_smth"], m["rcut"]
    x = torch.tensor(ext, dtype=torch.float64, requires_grad=True)
    jj = torch.tensor(nl, dtype=torch.long)
    mask = (jj >= 0).to(torch.float64)
    js = jj.clamp(min=0)
    d = x[js] - x[:nloc, None, :]
    d = torch.where(mask[..., None] > 0, d, torch.ones_like(d))
    r = torch.linalg.norm(d, dim=-1)
    u = (r - rs) / (rc - rs)
    sw = torch.where(r < rs, torch.ones_like(r),
                     torch.where(r >= rc, torch.zeros_like(r), u**3 * (-6 * u**2 + 15 * u - 10) + 1))
    R = torch.stack([sw / r, sw * d[..., 0] / r**2, sw * d[..., 1] / r**2, sw * d[..., 2] / r**2], -1)
    R = R * mask[..., None]
    types = torch.tensor(et[:nloc], dtype=torch.long)
    davg = torch.tensor(m["davg"])
    dstd = torch.tensor(m["dstd"])
    slot_type = np.concatenate([[t] * sel[t] for t in range(nt)])
    st = torch.tensor(slot_type, dtype=torch.long)
    Rn = (R - davg[types][:, st]) / dstd[types][:, st]
    G = torch.zeros(nloc, nnei, L3, dtype=torch.float64)
    for ti in range(nt):
        for tj in range(nt):
            P = torch.tensor(m["emb_params"][ti * nt + tj])
            layers, _ = _net_layers(P, [1, L1, L2], [L1, L2, L3])
            rows = types == ti
            s = Rn[rows][:, sec[tj]:sec[tj + 1], :1]
            h = s
            for W, b in layers:
                h = _act(h, W, b)
            G = G.index_put((rows.nonzero()[:, 0][:, None],
                             torch.arange(sec[tj], sec[tj + 1])[None, :]), h)
    T = torch.einsum("nsk,nsa->nka", Rn, G) / nnei
    D = torch.einsum("nka,nkb->nab", T, T[:, :, :M2]).reshape(nloc, L3 * M2)
    e = torch.zeros(nloc, dtype=torch.float64)
    Dn = L3 * M2
    F = m["fit"]
    for ti in range(nt):
        P = torch.tensor(m["fit_params"][ti])
        p = 0
        h = D[types == ti]
        for i, o in zip([Dn, F[0], F[1]], F):
            W = P[p:p + i * o].reshape(i, o); p += i * o
            b = P[p:p + o]; p += o
            idt = None
            if i == o:
                idt = P[p:p + o]; p += o
            h = _act(h, W, b, idt)
        Wo = P[p:p + F[2]]
        bo = P[p + F[2]]
        e = e.index_put((types == ti,), h @ Wo + bo + m["bias_atom_e"][ti])
    E = e.sum()
    g, = torch.autograd.grad(E, x)
    return e.detach().numpy(), (-g).numpy()


@pytest.mark.parametrize("case", ["water192", "hea1024"])
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
