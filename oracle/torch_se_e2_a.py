"""TEST INFRASTRUCTURE ONLY — a second, independent CPU restatement of the
DeepPot-SE `se_e2_a` evaluation, in torch fp64 with autograd forces.

Only tests/ (the cross-check of the C oracle, tests/test_torch_crosscheck.py)
and bench.py's cpu_baseline leg (a BLAS-backed CPU figure beside the scalar C
oracle's) use it; the shipped library never imports it. It is written from the
model's definition (DeepPot-SE, Zhang et al. 2018), not from the C oracle:
batched products over all slots of all centres of one type (the embedding and
fitting layers are matrix products on the host's BLAS), padded slots included
as DeePMD evaluates them, and forces by reverse-mode autograd instead of a
hand-written backward. The conventions it fixes are those of the C oracle
(oracle/se_e2_a.h): sel-sorted list with -1 padding, spline5 switch, env row
[s, s x/r, s y/r, s z/r] with s = sw(r)/r normalised by (davg, dstd) of the
(centre type, neighbour section), concat residual when a layer doubles its
width, per-neuron timestep on square fitting layers, energy head plus
bias_atom_e[type]. The force / virial assembly convention is that of the
reference's edge kernel (edge_force_virial.cu:1-14, :138-146).

Parity pin: tests/test_torch_crosscheck.py holds it to the C oracle (atom
energies 1e-12 eV, forces 1e-11 eV/A, virial 1e-9 eV) on several systems and
fitting shapes; the two were written independently, so an error in either
fails there.
"""
from __future__ import annotations

import numpy as np
import torch


def _act(x, W, b, idt=None):
    t = torch.tanh(x @ W + b)
    i, o = W.shape
    if o == i:
        return x + (idt * t if idt is not None else t)
    if o == 2 * i:
        return torch.cat([x, x], dim=-1) + t
    return t


def _emb_layers(params, L):
    """(W, b) of the embedding net 1 -> L1 -> L2 -> L3 from one parameter block."""
    out, p = [], 0
    for i, o in zip([1, L[0], L[1]], L):
        W = params[p:p + i * o].reshape(i, o); p += i * o
        b = params[p:p + o]; p += o
        out.append((W, b))
    return out


def _fit_layers(params, Dn, F):
    out, p = [], 0
    for i, o in zip([Dn, F[0], F[1]], F):
        W = params[p:p + i * o].reshape(i, o); p += i * o
        b = params[p:p + o]; p += o
        idt = None
        if i == o:
            idt = params[p:p + o]; p += o
        out.append((W, b, idt))
    return out, params[p:p + F[2]], params[p + F[2]]


class TorchSeA:
    """One model (the dict of the package's model format, or the C oracle's
    reader) with its parameters as torch fp64 tensors."""

    def __init__(self, m: dict):
        self.m = m
        self.nt = len(m["sel"])
        self.sel = list(m["sel"])
        self.sec = np.concatenate([[0], np.cumsum(self.sel)]).astype(int)
        self.nnei = int(self.sec[-1])
        self.L = list(m["emb"])
        self.M2 = int(m["axis"])
        self.F = list(m["fit"])
        nt = self.nt
        davg = np.asarray(m["davg"], np.float64).reshape(nt, nt, 4)
        dstd = np.asarray(m["dstd"], np.float64).reshape(nt, nt, 4)
        emb = np.asarray(m["emb_params"], np.float64).reshape(nt * nt, -1)
        fit = np.asarray(m["fit_params"], np.float64).reshape(nt, -1)
        # per-slot statistics of each centre type: [nt][nnei][4]
        slot_sec = np.concatenate([[t] * s for t, s in enumerate(self.sel)])
        self.davg = torch.tensor(davg[:, slot_sec, :])
        self.dstd = torch.tensor(dstd[:, slot_sec, :])
        self.emb = [[_emb_layers(torch.tensor(emb[ti * nt + tj]), self.L) for tj in range(nt)]
                    for ti in range(nt)]
        Dn = self.L[2] * self.M2
        self.fit = [_fit_layers(torch.tensor(fit[t]), Dn, self.F) for t in range(nt)]
        self.bias = np.asarray(m["bias_atom_e"], np.float64).reshape(nt)

    def energy(self, x, ext_type, nlist, nloc, first=0):
        """Atom energies of the centres first .. first + nloc - 1 of the
        extended system x ([nall, 3] tensor), whose neighbour rows are nlist
        ([nloc, nnei]); differentiable in x."""
        rs, rc = float(self.m["rcut_smth"]), float(self.m["rcut"])
        jj = torch.as_tensor(np.asarray(nlist), dtype=torch.long)
        mask = (jj >= 0).to(torch.float64)
        d = x[jj.clamp(min=0)] - x[first:first + nloc, None, :]
        d = torch.where(mask[..., None] > 0, d, torch.ones_like(d))
        r = torch.linalg.norm(d, dim=-1)
        u = (r - rs) / (rc - rs)
        sw = torch.where(r < rs, torch.ones_like(r),
                         torch.where(r >= rc, torch.zeros_like(r),
                                     u ** 3 * (-6 * u ** 2 + 15 * u - 10) + 1))
        R = torch.stack([sw / r, sw * d[..., 0] / r ** 2, sw * d[..., 1] / r ** 2,
                         sw * d[..., 2] / r ** 2], -1) * mask[..., None]
        ti_all = np.asarray(ext_type[first:first + nloc])
        e = torch.zeros(nloc, dtype=torch.float64)
        L3, M2 = self.L[2], self.M2
        for ti in range(self.nt):
            rows = np.nonzero(ti_all == ti)[0]
            if len(rows) == 0:
                continue
            ridx = torch.as_tensor(rows, dtype=torch.long)
            Rn = (R[ridx] - self.davg[ti]) / self.dstd[ti]          # [n, nnei, 4]
            G = []
            for tj in range(self.nt):
                h = Rn[:, self.sec[tj]:self.sec[tj + 1], :1]
                for W, b in self.emb[ti][tj]:
                    h = _act(h, W, b)
                G.append(h)
            G = torch.cat(G, dim=1)                                  # [n, nnei, L3]
            T = torch.bmm(Rn.transpose(1, 2), G) / self.nnei         # [n, 4, L3]
            D = torch.bmm(T.transpose(1, 2), T[:, :, :M2].contiguous()).reshape(len(rows), L3 * M2)
            layers, Wo, bo = self.fit[ti]
            h = D
            for W, b, idt in layers:
                h = _act(h, W, b, idt)
            e = e.index_put((ridx,), h @ Wo + bo + float(self.bias[ti]))
        return e

    def evaluate(self, ext, ext_type, nlist, nloc, chunk=128):
        """(atom energies [nloc], forces [nall, 3]) over the extended system:
        F = -dE/dx by autograd, ghost contributions left in ghost rows. The
        centres go through in chunks of `chunk` (one graph each, gradients
        accumulated), which keeps every intermediate in the host's caches."""
        x = torch.tensor(np.asarray(ext, np.float64), requires_grad=True)
        nl = np.asarray(nlist)
        es = []
        for c0 in range(0, nloc, chunk):
            c1 = min(nloc, c0 + chunk)
            e = self.energy(x, ext_type, nl[c0:c1], c1 - c0, first=c0)
            e.sum().backward()
            es.append(e.detach())
        es = torch.cat(es) if es else torch.zeros(0, dtype=torch.float64)
        g = x.grad if x.grad is not None else torch.zeros_like(x)
        return es.numpy(), (-g).numpy()


def torch_eval(m, ext, et, nl, nloc):
    """Atom energies and extended-system forces of model dict m."""
    return TorchSeA(m).evaluate(ext, et, nl, nloc)
