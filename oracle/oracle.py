"""TEST INFRASTRUCTURE ONLY — ctypes front end of the CPU oracle (liborc.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker / CPU baseline; the shipped library never
imports it. The model reader below is the oracle's own, independent of the
package's loader, so a loader bug shows up as a parity failure.

Parity pins of each function (what fixes it besides retyping the formula):
  ghosts / candidates  brute force == cell list; periodic-image invariance
  format_nlist         hand-built ties, exact-rcut atoms, sel overflow by one
  switch / env_mat     closed forms at rs, rc; C2 continuity; finite differences
  eval (nets, D, fit)  independent torch fp64 autograd restatement
  eval (backward)      F = -dE/dx and W = -dE/d(strain) by central differences
  eval (force/virial)  sum F = 0, W symmetric, W = sum atom_virial
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

MAX_TYPES = 8


class OrcModel(C.Structure):
    _fields_ = [("ntypes", C.c_int), ("nnei", C.c_int), ("sel", C.c_int * MAX_TYPES),
                ("sec", C.c_int * (MAX_TYPES + 1)), ("rcut", C.c_double), ("rcut_smth", C.c_double),
                ("emb", C.c_int * 3), ("axis", C.c_int), ("fit", C.c_int * 3),
                ("davg", C.c_void_p), ("dstd", C.c_void_p), ("emb_params", C.c_void_p),
                ("fit_params", C.c_void_p), ("bias_atom_e", C.c_void_p)]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liborc.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(path)
        P = C.c_void_p
        L.orc_ghost_count.argtypes = [C.c_int, P, P, C.c_double]
        L.orc_build_ghosts.argtypes = [C.c_int, P, P, P, C.c_double, C.c_int, P, P, P]
        L.orc_candidates_brute.argtypes = [C.c_int, C.c_int, P, P, C.c_double, C.c_long, P, P]
        L.orc_candidates_brute.restype = C.c_long
        L.orc_candidates_cell.argtypes = [C.c_int, C.c_int, P, P, P, C.c_double, C.c_long, P, P]
        L.orc_candidates_cell.restype = C.c_long
        L.orc_format_nlist.argtypes = [P, C.c_int, P, P, P, P, P]
        L.orc_env_mat.argtypes = [P, C.c_int, P, P, P, P, P, P]
        L.orc_switch.argtypes = [C.c_double, C.c_double, C.c_double, C.POINTER(C.c_double)]
        L.orc_switch.restype = C.c_double
        L.orc_embed.argtypes = [P, C.c_int, C.c_int, C.c_double, P]
        L.orc_eval.argtypes = [P, C.c_int, C.c_int, P, P, P, C.c_int, P, P, P, P, P, P, P, P]
        L.orc_fold.argtypes = [C.c_int, C.c_int, P, P, P, P, P]
        L.orc_prod_force.argtypes = [C.c_int, C.c_int, C.c_int, P, P, P, P, P, P]
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def read_model_bytes(buf: bytes) -> dict:
    """Independent reader of the DPAMDSEA model layout (see the package's model.py)."""
    assert buf[:8] == b"DPAMDSEA", "bad magic"
    off = 8
    ver, nt = struct.unpack_from("<II", buf, off); off += 8
    assert ver == 1
    sel = list(struct.unpack_from(f"<{nt}I", buf, off)); off += 4 * nt
    rcut, rs = struct.unpack_from("<dd", buf, off); off += 16
    emb = list(struct.unpack_from("<3I", buf, off)); off += 12
    (axis,) = struct.unpack_from("<I", buf, off); off += 4
    fit = list(struct.unpack_from("<3I", buf, off)); off += 16
    off += 16 * nt
    vals = np.frombuffer(buf, dtype="<f8", offset=off)
    L1, L2, L3 = emb
    eb = 2 * L1 + L1 * L2 + L2 + L2 * L3 + L3
    ins = [L3 * axis, fit[0], fit[1]]
    fb = sum(i * o + o + (o if i == o else 0) for i, o in zip(ins, fit)) + fit[2] + 1
    q = 0

    def take(n):
        nonlocal q
        a = np.array(vals[q:q + n], dtype=np.float64)
        q += n
        return a
    m = dict(ntypes=nt, sel=sel, rcut=rcut, rcut_smth=rs, emb=emb, axis=axis, fit=fit,
             davg=take(nt * nt * 4), dstd=take(nt * nt * 4), emb_params=take(nt * nt * eb),
             fit_params=take(nt * fb), bias_atom_e=take(nt))
    assert q == len(vals), "trailing bytes in model file"
    return m


class Oracle:
    """fp64 CPU evaluation of one model."""

    def __init__(self, model_bytes: bytes):
        self.m = read_model_bytes(model_bytes)
        m = self.m
        s = OrcModel()
        s.ntypes = m["ntypes"]
        s.nnei = sum(m["sel"])
        acc = 0
        for t in range(m["ntypes"]):
            s.sel[t] = m["sel"][t]
            s.sec[t] = acc
            acc += m["sel"][t]
        s.sec[m["ntypes"]] = acc
        s.rcut, s.rcut_smth = m["rcut"], m["rcut_smth"]
        for k in range(3):
            s.emb[k] = m["emb"][k]
            s.fit[k] = m["fit"][k]
        s.axis = m["axis"]
        s.davg, s.dstd = _p(m["davg"]), _p(m["dstd"])
        s.emb_params, s.fit_params = _p(m["emb_params"]), _p(m["fit_params"])
        s.bias_atom_e = _p(m["bias_atom_e"])
        self.s = s
        self.nnei = s.nnei
        self.sec = [s.sec[t] for t in range(m["ntypes"] + 1)]
        self.ndescrpt = m["emb"][2] * m["axis"]

    @property
    def ref(self):
        return C.byref(self.s)

    # ---- geometry -------------------------------------------------------
    @staticmethod
    def ghosts(coord, atype, box, rcut):
        coord = np.ascontiguousarray(coord, np.float64)
        atype = np.ascontiguousarray(atype, np.int32)
        box = np.ascontiguousarray(box, np.float64)
        nloc = len(atype)
        n = lib().orc_ghost_count(nloc, _p(coord), _p(box), rcut)
        if n < 0:
            raise ValueError("box must be lower-triangular with positive diagonal")
        ext = np.zeros((n, 3))
        et = np.zeros(n, np.int32)
        mp = np.zeros(n, np.int32)
        r = lib().orc_build_ghosts(nloc, _p(coord), _p(atype), _p(box), rcut, n, _p(ext), _p(et), _p(mp))
        assert r == n
        return ext, et, mp

    @staticmethod
    def candidates(nloc, ext, etype, rc, method="cell", box=None):
        ext = np.ascontiguousarray(ext, np.float64)
        etype = np.ascontiguousarray(etype, np.int32)
        off = np.zeros(nloc + 1, np.int64)
        fn = lib().orc_candidates_cell if method == "cell" else lib().orc_candidates_brute
        args = [nloc, len(etype), _p(ext), _p(etype)]
        if method == "cell":
            args.append(None)
        n = fn(*args, rc, 0, _p(off), None)
        cand = np.zeros(max(n, 1), np.int32)
        n2 = fn(*args, rc, n, _p(off), _p(cand))
        assert n2 == n
        return off, cand[:n]

    def format_nlist(self, nloc, ext, etype, off, cand):
        nl = np.full((nloc, self.nnei), -1, np.int32)
        lib().orc_format_nlist(self.ref, nloc, _p(np.ascontiguousarray(ext)), _p(etype), _p(off),
                               _p(cand), _p(nl))
        return nl

    def env_mat(self, nloc, ext, etype, nlist):
        env = np.zeros((nloc, self.nnei, 4))
        envd = np.zeros((nloc, self.nnei, 4, 3))
        rij = np.zeros((nloc, self.nnei, 3))
        lib().orc_env_mat(self.ref, nloc, _p(ext), _p(etype), _p(nlist), _p(env), _p(envd), _p(rij))
        return env, envd, rij

    def embed(self, ti, tj, s):
        g = np.zeros(self.m["emb"][2])
        lib().orc_embed(self.ref, ti, tj, float(s), _p(g))
        return g

    def switch(self, r):
        d = C.c_double()
        v = lib().orc_switch(float(r), self.m["rcut_smth"], self.m["rcut"], C.byref(d))
        return v, d.value

    # ---- evaluation -----------------------------------------------------
    def eval_ext(self, nloc, ext, etype, nlist, nthreads=0, want_atomic=True, want_internals=False):
        ext = np.ascontiguousarray(ext, np.float64)
        etype = np.ascontiguousarray(etype, np.int32)
        nlist = np.ascontiguousarray(nlist, np.int32)
        nall = len(etype)
        ae = np.zeros(nloc)
        f = np.zeros((nall, 3))
        v = np.zeros(9)
        av = np.zeros((nall, 9)) if want_atomic else None
        eg = np.zeros((nloc, self.nnei, 3))
        d = dd = nd = None
        if want_internals:
            d = np.zeros((nloc, self.ndescrpt))
            dd = np.zeros((nloc, self.ndescrpt))
            nd = np.zeros((nloc, self.nnei, 4))
        r = lib().orc_eval(self.ref, nloc, nall, _p(ext), _p(etype), _p(nlist), nthreads, _p(ae),
                           _p(d), _p(dd), _p(nd), _p(eg), _p(f), _p(v), _p(av))
        assert r == 0
        out = dict(energy=float(ae.sum()), atom_energy=ae, force=f, virial=v, atom_virial=av,
                   edge_grad=eg)
        if want_internals:
            out.update(descrpt=d, dE_dD=dd, net_deriv=nd)
        return out

    def prod_force(self, nloc, ext, nlist, edge_grad, mapping=None):
        """ProdForce / ProdVirial of given per-slot edge gradients (the
        oracle's own assembly, orc_prod_force). Over the extended atoms, or,
        with `mapping`, folded onto the nloc owners (orc_fold)."""
        ext = np.ascontiguousarray(ext, np.float64)
        nlist = np.ascontiguousarray(nlist, np.int32)
        eg = np.ascontiguousarray(edge_grad, np.float64)
        nall = len(ext)
        assert nlist.shape == (nloc, self.nnei) and eg.shape == (nloc, self.nnei, 3)
        assert nlist.max(initial=-1) < nall
        f = np.zeros((nall, 3))
        v = np.zeros(9)
        av = np.zeros((nall, 9))
        lib().orc_prod_force(nloc, nall, self.nnei, _p(ext), _p(nlist), _p(eg), _p(f), _p(v), _p(av))
        if mapping is None:
            return f, v, av
        mp = np.ascontiguousarray(mapping, np.int32)
        assert len(mp) == nall
        f2 = np.zeros((nloc, 3))
        av2 = np.zeros((nloc, 9))
        lib().orc_fold(nloc, nall, _p(mp), _p(f), _p(av), _p(f2), _p(av2))
        return f2, v, av2

    def neighbor_list(self, coord, atype, box):
        """Ghosts + cell-list candidates + sel formatting for a periodic box."""
        ext, et, mp = self.ghosts(coord, atype, box, self.m["rcut"])
        nloc = len(atype)
        off, cand = self.candidates(nloc, ext, et, self.m["rcut"], "cell")
        nl = self.format_nlist(nloc, ext, et, off, cand)
        return ext, et, mp, nl

    def compute(self, coord, atype, box, nthreads=0, want_internals=False):
        """Standalone periodic evaluation (mirrors DeepPot::compute(coord, atype, box)):
        ghost forces and atom virials folded onto their owners."""
        ext, et, mp, nl = self.neighbor_list(coord, atype, box)
        nloc = len(atype)
        out = self.eval_ext(nloc, ext, et, nl, nthreads, True, want_internals)
        f = np.zeros((nloc, 3))
        av = np.zeros((nloc, 9))
        lib().orc_fold(nloc, len(et), _p(mp), _p(out["force"]), _p(out["atom_virial"]), _p(f), _p(av))
        out.update(force=f, atom_virial=av, nlist=nl, ext_coord=ext, ext_type=et, mapping=mp)
        return out
