"""TEST INFRASTRUCTURE ONLY — fp64 CPU restatement of the DPA4C-Nano model.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker / CPU baseline; the shipped library never
imports it. It reads model files with its own reader, independent of the
package's loader, and evaluates everything in float64 with torch on the CPU;
edge gradients come from autograd, so the backward is the exact derivative of
the forward written here, independent of the analytic backward of the HIP
kernels.

What each part restates (reference files under dpa4c-runtime/):
  edge geometry   r = sqrt(|d|^2 + eps^2), u = d / r, d = x_src - x_dst
                  (include/dpa_chain/graph_compress.cuh:220-241,
                  components/deepmd-op/overlays/op/pt/dpa4c/raw_geometry.cuh:5-22)
  envelope        C3 polynomial c3(r) (graph_compress.cuh:218-227)
  radial table    quintic per interval, x = r - i*stride, i = min(floor(r /
                  stride), n - 1) on the canonical path (graph_compress.cuh:92-125)
  PairFiLM        film = a * radial + b per (centre type, neighbour type);
                  amplitude = film * env, angular = amplitude * env
                  (graph_compress_kernel.cuh:235-259)
  harmonics       [1, u, sqrt3 xy, sqrt3 yz, (3z^2-1)/2, sqrt3 xz,
                  sqrt3/2 (x^2-y^2)] (graph_compress.cuh:265-277)
  moments         scalar / vector / tensor sums and the two envelope masses,
                  normalised by rsqrt(mass + degree_floor)
                  (graph_compress_kernel.cuh:310-418)
  readout         alignment and probe matrices, Gram blocks with sqrt2 off the
                  diagonal, Bis112 = -1/sqrt5 l^T STF(p) r, Bis222 = kappa
                  tr(ABC), Quartic = |STF(p) v|^2, divisors, type embedding,
                  standardisation (graph_compress_kernel.cuh:494-690,
                  graph_compress.cuh:566-600, 622-636)
  fitting         h = act(h W + b) (+ h on square resnet layers), e = h w +
                  b_head + bias_atom_e[type] (op/pt/graph_fitting.cu:1-25)
  force / virial  force[dst] += g, force[src] -= g, atom_virial[src] +=
                  -g (x) d (op/pt/edge_force_virial.cu:1-14, 138-146)

Parity pins (tests/test_dpa4c_oracle.py): closed forms of every readout block
for one and two edges with identity readout matrices; the C3 envelope's value
and derivatives at 0 and rcut; C2 continuity of the radial table across
knots; |Y2(u)| = 1 and STF(Y2(u)) = sqrt(3/2)(uu^T - I/3); rotation,
translation and permutation invariance of all 70 descriptor entries; F =
-dE/dx and W = -dE/d(strain) by central differences; sum F = 0; the
magnitudes of the Bis112 and Bis222 couplings (1/sqrt5, sqrt(12/35)) as the
unit-Frobenius normalisations of the Cartesian Gaunt tensors in the packed
STF basis. Their signs are the reference's convention
(graph_compress.cuh:34-38, graph_compress_kernel.cuh:581-584) and are pinned
only by that citation: parity unpinned for the two signs.
"""
from __future__ import annotations

import math
import struct

import numpy as np
import torch

from .oracle import Oracle

KAPPA_222 = -0.58554004376911988
SQ2, SQ3, SQ5, SQ6 = math.sqrt(2.0), math.sqrt(3.0), math.sqrt(5.0), math.sqrt(6.0)
C0, C1, C2, K1, K2 = 8, 4, 4, 4, 2
OUT_WIDTH = 70


def read_model_bytes(buf: bytes) -> dict:
    """Independent reader of the DPAMDC4N layout (see the package's dpa4c.py)."""
    assert buf[:8] == b"DPAMDC4N", "bad magic"
    off = 8
    ver, nt = struct.unpack_from("<II", buf, off); off += 8
    assert ver == 1
    sel = list(struct.unpack_from(f"<{nt}I", buf, off)); off += 4 * nt
    rcut, eps, floor, stride = struct.unpack_from("<4d", buf, off); off += 32
    n_int, ch, lmax = struct.unpack_from("<3I", buf, off); off += 12
    assert (ch, lmax) == (C0, 2)
    (nl,) = struct.unpack_from("<I", buf, off); off += 4
    fit = list(struct.unpack_from(f"<{nl}I", buf, off)); off += 4 * nl
    act, resnet = struct.unpack_from("<II", buf, off); off += 8
    off += 16 * nt

    def take(n, dt="<f4"):
        nonlocal off
        a = np.frombuffer(buf, dtype=dt, count=n, offset=off).astype(np.float64)
        off += np.dtype(dt).itemsize * n
        return a
    m = dict(ntypes=nt, sel=sel, rcut=rcut, eps=eps, floor=floor, stride=stride, n_int=n_int,
             fit=fit, act=act, resnet=resnet)
    m["table"] = take(n_int * 6 * C0).reshape(n_int, 6, C0)
    m["film"] = take(nt * nt * C0 * 2).reshape(nt * nt, C0, 2)
    m["Ma"] = take(C1 * C1).reshape(C1, C1)
    m["Mt"] = take(C2 * C2).reshape(C2, C2)
    m["Pv"] = take(C1 * K1).reshape(C1, K1)
    m["Pt"] = take(C2 * K2).reshape(C2, K2)
    m["temb"] = take(nt * C0).reshape(nt, C0)
    m["mean"], m["inv_std"] = take(OUT_WIDTH), take(OUT_WIDTH)
    layers, din = [], OUT_WIDTH
    for w in fit:
        layers.append((take(din * w).reshape(din, w), take(w)))
        din = w
    m["layers"] = layers
    m["w_head"] = take(din)
    m["b_head"] = float(take(1)[0])
    m["bias"] = take(nt, "<f8")
    assert off == len(buf), "trailing bytes in model file"
    return m


def upper_pairs(width):
    """(row, column) of the row-major upper triangle, diagonal included
    (decode_upper_pair, graph_compress.cuh:556-564)."""
    return [(r, c) for r in range(width) for c in range(r, width)]


def stf(p):
    """Packed degree-two components [..., 5] -> symmetric traceless [..., 3, 3]
    (packed_to_stf, graph_compress.cuh:520-530)."""
    m00 = -p[..., 2] / SQ6 + p[..., 4] / SQ2
    m11 = -p[..., 2] / SQ6 - p[..., 4] / SQ2
    m22 = 2.0 * p[..., 2] / SQ6
    m01, m12, m02 = p[..., 0] / SQ2, p[..., 1] / SQ2, p[..., 3] / SQ2
    return torch.stack([torch.stack([m00, m01, m02], -1), torch.stack([m01, m11, m12], -1),
                        torch.stack([m02, m12, m22], -1)], -2)


def envelope(r, rcut):
    """C3 envelope: with u = clamp((rcut - r)/rcut, 0, 1), x = 1 - u,
    env = u^4 (1 + 4x + 10x^2 + 20x^3 + 35x^4) (graph_compress.cuh:218-225)."""
    u = torch.clamp((rcut - r) / rcut, 0.0, 1.0)
    x = 1.0 - u
    return u ** 4 * (1.0 + x * (4.0 + x * (10.0 + x * (20.0 + 35.0 * x))))


def harmonics2(u):
    """Degree-two real Cartesian harmonics of a direction [E, 3] -> [E, 5]
    (fill_angular_basis, graph_compress.cuh:265-277)."""
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    return torch.stack([SQ3 * x * y, SQ3 * y * z, 0.5 * (3.0 * z * z - 1.0), SQ3 * x * z,
                        0.5 * SQ3 * (x * x - y * y)], 1)


class Dpa4cOracle:
    """fp64 CPU evaluation of one DPA4C-Nano model."""

    def __init__(self, model_bytes: bytes):
        self.m = read_model_bytes(model_bytes)
        t = lambda a: torch.as_tensor(a, dtype=torch.float64)  # noqa: E731
        m = self.m
        self.T = {k: t(m[k]) for k in ("table", "film", "Ma", "Mt", "Pv", "Pt", "temb", "mean",
                                       "inv_std", "w_head", "bias")}
        self.layers = [(t(W), t(b)) for W, b in m["layers"]]

    # ---- descriptor -----------------------------------------------------
    def radial(self, r):
        m = self.m
        idx = torch.clamp(torch.floor(r.detach() / m["stride"]).long(), max=m["n_int"] - 1)
        x = r - idx.to(torch.float64) * m["stride"]
        c = self.T["table"][idx]                                   # [E, 6, C0]
        out = c[:, 5]
        for k in range(4, -1, -1):
            out = c[:, k] + out * x[:, None]
        return out

    def moments(self, ev, src, dst, atype, n_nodes):
        """Raw moment sums of every destination node: scalar [N, C0], vector
        [N, 3, C1], tensor [N, 5, C2], masses [N] (sum env^2, sum env^4)."""
        m = self.m
        nt = m["ntypes"]
        sq = (ev * ev).sum(1) + m["eps"] ** 2
        r = torch.sqrt(sq)
        u = ev / r[:, None]
        env = envelope(r, m["rcut"])
        rad = self.radial(r)
        pair = atype[dst] * nt + atype[src]
        film = self.T["film"][pair]                                # [E, C0, 2]
        amp = (film[..., 0] * rad + film[..., 1]) * env[:, None]
        ang = amp * env[:, None]
        Y2 = harmonics2(u)
        z = lambda *s: torch.zeros(*s, dtype=torch.float64)  # noqa: E731
        scal = z(n_nodes, C0).index_add(0, dst, amp)
        vec = z(n_nodes, 3, C1).index_add(0, dst, u[:, :, None] * ang[:, None, :C1])
        ten = z(n_nodes, 5, C2).index_add(0, dst, Y2[:, :, None] * ang[:, None, :C2])
        ms = z(n_nodes).index_add(0, dst, env ** 2)
        ma = z(n_nodes).index_add(0, dst, env ** 4)
        return scal, vec, ten, ms, ma

    def readout(self, scal, vec, ten, ms, ma, node_type):
        """Raw (unstandardised) 70-wide descriptor from the raw moments."""
        T, fl = self.T, self.m["floor"]
        ns, na = (ms + fl) ** -0.5, (ma + fl) ** -0.5
        s = scal * ns[:, None]
        v = vec * na[:, None, None]
        t = ten * na[:, None, None]
        av, at = v @ T["Ma"], t @ T["Mt"]
        pv, pt = av @ T["Pv"], at @ T["Pt"]                         # [N,3,K1], [N,5,K2]
        g1 = [(av[:, :, r] * av[:, :, c]).sum(1) * (1.0 if r == c else SQ2)
              for r, c in upper_pairs(C1)]
        g2 = [(at[:, :, r] * at[:, :, c]).sum(1) * (1.0 if r == c else SQ2)
              for r, c in upper_pairs(C2)]
        S = [stf(pt[:, :, k]) for k in range(K2)]                   # [N,3,3] each
        b112 = []
        pairs1 = upper_pairs(K1)
        for o in range(len(pairs1) * K2):
            k = o % K2
            f, sc = pairs1[o // K2]
            val = -(pv[:, :, f] * (S[k] @ pv[:, :, sc, None])[..., 0]).sum(1) / SQ5
            b112.append(val * (1.0 if f == sc else SQ2))
        b222 = []
        for (a, b, c), w in zip(((0, 0, 0), (0, 0, 1), (0, 1, 1), (1, 1, 1)), (1.0, SQ3, SQ3, 1.0)):
            prod = S[a] @ S[b] @ S[c]
            b222.append(KAPPA_222 * w * prod.diagonal(dim1=-2, dim2=-1).sum(-1))
        quart = []
        for o in range(K1 * K2):
            vi, ti = o % K1, o // K1
            w = (S[ti] @ pv[:, :, vi, None])[..., 0]
            quart.append((w * w).sum(1))
        blocks = [s] + [torch.stack(b, 1) for b in (g1, g2, b112, b222, quart)]
        blocks.append(torch.stack([torch.sqrt(ms + fl), torch.sqrt(ma + fl)], 1))
        blocks.append(T["temb"][node_type])
        raw = torch.cat(blocks, 1)
        assert raw.shape[1] == OUT_WIDTH
        return raw

    def descriptor(self, ev, src, dst, atype, n_nodes, standardise=True):
        raw = self.readout(*self.moments(ev, src, dst, atype, n_nodes), atype[:n_nodes])
        if not standardise:
            return raw
        return (raw - self.T["mean"]) * self.T["inv_std"]

    def fitting(self, D, node_type):
        m = self.m
        h = D
        for li, (W, b) in enumerate(self.layers):
            pre = h @ W + b
            y = torch.tanh(pre) if m["act"] == 0 else pre * torch.sigmoid(pre)
            if (m["resnet"] >> li) & 1 and W.shape[0] == W.shape[1]:
                y = y + h
            h = y
        return h @ self.T["w_head"] + m["b_head"] + self.T["bias"][node_type]

    # ---- evaluation -----------------------------------------------------
    def evaluate_graph(self, atype, src, dst, edge_vec, nloc, nall, want_internals=False):
        """The canonical-graph contract: edges (src -> dst, dst < nloc) with
        vectors d = x_src - x_dst; returns atom_energy [nloc], edge_grad
        [E, 3] = dE/dd, force [nall, 3] and atom_virial [nall, 9] unfolded
        (ghost slots keep their own), virial [9], energy."""
        at = torch.as_tensor(np.asarray(atype), dtype=torch.long)
        s = torch.as_tensor(np.asarray(src), dtype=torch.long)
        d = torch.as_tensor(np.asarray(dst), dtype=torch.long)
        ev = torch.as_tensor(np.asarray(edge_vec, np.float64)).clone().requires_grad_(True)
        # virtual atoms (type < 0) carry no energy; callers give them no edges
        real = at[:nloc] >= 0
        atc = torch.clamp(at, min=0)
        D = self.descriptor(ev, s, d, atc, nloc)
        e = torch.where(real, self.fitting(D, atc[:nloc]), torch.zeros((), dtype=torch.float64))
        E = e.sum()
        g = torch.autograd.grad(E, ev)[0] if len(s) else torch.zeros((0, 3), dtype=torch.float64)
        g = g.numpy()
        evn = ev.detach().numpy()
        f = np.zeros((nall, 3))
        np.add.at(f, np.asarray(dst), g)
        np.add.at(f, np.asarray(src), -g)
        av = np.zeros((nall, 9))
        np.add.at(av, np.asarray(src), -(g[:, :, None] * evn[:, None, :]).reshape(-1, 9))
        out = dict(energy=float(E.detach()), atom_energy=e.detach().numpy(), edge_grad=g,
                   force=f, atom_virial=av, virial=av.sum(0))
        if want_internals:
            out["descriptor"] = D.detach().numpy()
        return out

    def edges(self, coord, atype, box):
        """Standalone graph of a periodic (or open, box None) system: ghosts,
        then every (i local, j extended) pair with r^2 < rcut^2 (strict, the
        reference's cutoff predicate, exact_cut.cuh:10-20), d = x_j - x_i."""
        rc = self.m["rcut"]
        coord = np.ascontiguousarray(coord, np.float64).reshape(-1, 3)
        atype = np.asarray(atype, np.int32)
        nloc = len(atype)
        if box is None:
            ext, et, mp = coord.copy(), atype.copy(), np.arange(nloc, dtype=np.int32)
        else:
            ext, et, mp = Oracle.ghosts(coord, atype, box, rc)
        off, cand = Oracle.candidates(nloc, ext, et, rc, "brute")
        dst = np.repeat(np.arange(nloc), np.diff(off))
        src = cand.astype(np.int64)
        dv = ext[src] - ext[dst]
        r2 = dv[:, 0] * dv[:, 0] + dv[:, 1] * dv[:, 1] + dv[:, 2] * dv[:, 2]
        keep = r2 < rc * rc
        return ext, et, mp, src[keep], dst[keep], dv[keep]

    def compute(self, coord, atype, box, want_internals=False):
        """DeepPot::compute(coord, atype, box) semantics: ghost forces and atom
        virials folded onto their owners."""
        ext, et, mp, src, dst, dv = self.edges(coord, atype, box)
        nloc = len(atype)
        out = self.evaluate_graph(et, src, dst, dv, nloc, len(et), want_internals)
        f = np.zeros((nloc, 3))
        av = np.zeros((nloc, 9))
        np.add.at(f, mp, out["force"])
        np.add.at(av, mp, out["atom_virial"])
        out.update(force=f, atom_virial=av, src=src, dst=dst, edge_vec=dv, ext_coord=ext,
                   ext_type=et, mapping=mp)
        return out
