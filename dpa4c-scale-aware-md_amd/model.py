"""se_e2_a model files: seeded random initialisation, writer and reader.

File layout (little endian), read by the C++ loader in csrc/model.cpp:

    8 bytes  magic "DPAMDSEA"
    u32      version (1)
    u32      ntypes
    u32[nt]  sel
    f64      rcut, rcut_smth
    u32[3]   embedding widths L1, L2, L3
    u32      axis (M2)
    u32[3]   fitting widths F0, F1, F2
    u32      precision the model is evaluated in: 0 fp64, 1 mixed (fp32
             nets, fp64 env matrix, forces, virials); files written while
             this word was reserved read as fp64
    char[nt][16] type_map, NUL padded
    f64[nt][nt][4] davg     (per centre type, per neighbour section)
    f64[nt][nt][4] dstd
    f64[nt*nt][emb_block]   embedding net of pair (ti, tj) at index ti*nt + tj:
                            W1[1,L1] b1[L1] W2[L1,L2] b2[L2] W3[L2,L3] b3[L3]
    f64[nt][fit_block]      fitting net of centre type t: for k = 0..2
                            W_k[in,out] b_k[out] (idt_k[out] iff out == in),
                            then Wo[F2] bo[1]; in_0 = L3*axis
    f64[nt]  bias_atom_e

Weights are row-major [in, out]. The metadata keys mirror what the
reference's model API reads from a model (rcut, ntypes/type_map, sel:
deepmd-op/overlays/api_cc/src/DeepPotPTExpt.cc:368-478).
"""
from __future__ import annotations

import struct

import numpy as np

from .systems import Stream

MAGIC = b"DPAMDSEA"

KINDS = {
    "water": dict(type_map=["O", "H"], sel=[46, 92], rcut=6.0, rcut_smth=0.5,
                  emb=[25, 50, 100], axis=16, fit=[240, 240, 240]),
    "cu": dict(type_map=["Cu"], sel=[138], rcut=8.0, rcut_smth=2.0,
               emb=[32, 64, 128], axis=16, fit=[240, 240, 240]),
    "hea": dict(type_map=["Co", "Cr", "Fe", "Ni"], sel=[40, 40, 40, 40], rcut=6.0,
                rcut_smth=0.5, emb=[32, 64, 128], axis=16, fit=[240, 240, 240]),
}


def emb_block_size(emb):
    L1, L2, L3 = emb
    return L1 + L1 + L1 * L2 + L2 + L2 * L3 + L3


def fit_shapes(emb, axis, fit):
    ins = [emb[2] * axis, fit[0], fit[1]]
    return list(zip(ins, fit))


def fit_block_size(emb, axis, fit):
    n = 0
    for i, o in fit_shapes(emb, axis, fit):
        n += i * o + o + (o if o == i else 0)
    return n + fit[2] + 1


def random_model(kind: str, seed: int, **overrides) -> dict:
    """Seeded random-init weights: W ~ N(0, 1/(in+out)), b ~ N(0, 1),
    idt ~ N(0.1, 0.001^2), bias_atom_e ~ N(0, 1); davg nonzero only in column 0
    and dstd > 0, both constant per (centre type, neighbour section)."""
    spec = dict(KINDS[kind])
    spec.update(overrides)
    nt = len(spec["type_map"])
    emb, axis, fit = spec["emb"], spec["axis"], spec["fit"]
    st = Stream(seed, 7)
    blocks = []
    for _ in range(nt * nt):
        parts = []
        ins = [1, emb[0], emb[1]]
        for i, o in zip(ins, emb):
            parts.append(st.normal(i * o) / np.sqrt(i + o))
            parts.append(st.normal(o))
        blocks.append(np.concatenate(parts))
    emb_params = np.stack(blocks)
    fblocks = []
    for _ in range(nt):
        parts = []
        for i, o in fit_shapes(emb, axis, fit):
            parts.append(st.normal(i * o) / np.sqrt(i + o))
            parts.append(st.normal(o))
            if o == i:
                parts.append(0.1 + 0.001 * st.normal(o))
        parts.append(st.normal(fit[2]) / np.sqrt(fit[2] + 1))
        parts.append(st.normal(1))
        fblocks.append(np.concatenate(parts))
    fit_params = np.stack(fblocks)
    davg = np.zeros((nt, nt, 4))
    dstd = np.zeros((nt, nt, 4))
    davg[:, :, 0] = 0.1 + 0.02 * st.normal(nt * nt).reshape(nt, nt)
    dstd[:, :, 0] = 0.1 * (1.0 + 0.1 * np.abs(st.normal(nt * nt))).reshape(nt, nt)
    dstd[:, :, 1:] = (0.15 * (1.0 + 0.1 * np.abs(st.normal(nt * nt)))).reshape(nt, nt, 1)
    bias = st.normal(nt)
    assert emb_params.shape[1] == emb_block_size(emb)
    assert fit_params.shape[1] == fit_block_size(emb, axis, fit)
    return dict(type_map=list(spec["type_map"]), sel=list(spec["sel"]), rcut=float(spec["rcut"]),
                rcut_smth=float(spec["rcut_smth"]), emb=list(emb), axis=int(axis), fit=list(fit),
                davg=davg, dstd=dstd, emb_params=emb_params, fit_params=fit_params,
                bias_atom_e=bias)


def to_bytes(m: dict) -> bytes:
    nt = len(m["type_map"])
    out = [MAGIC, struct.pack("<II", 1, nt), struct.pack(f"<{nt}I", *m["sel"]),
           struct.pack("<dd", m["rcut"], m["rcut_smth"]), struct.pack("<3I", *m["emb"]),
           struct.pack("<I", m["axis"]), struct.pack("<3I", *m["fit"]),
           struct.pack("<I", 1 if m.get("precision", "fp64") == "mixed" else 0)]
    for name in m["type_map"]:
        b = name.encode()[:15]
        out.append(b + b"\0" * (16 - len(b)))
    for key in ("davg", "dstd", "emb_params", "fit_params", "bias_atom_e"):
        out.append(np.ascontiguousarray(m[key], dtype="<f8").tobytes())
    return b"".join(out)


def write_model(path: str, m: dict) -> str:
    with open(path, "wb") as f:
        f.write(to_bytes(m))
    return path


def from_bytes(buf: bytes) -> dict:
    if buf[:8] != MAGIC:
        raise ValueError("not a DPAMDSEA model file")
    off = 8
    ver, nt = struct.unpack_from("<II", buf, off); off += 8
    if ver != 1:
        raise ValueError(f"unsupported model version {ver}")
    sel = list(struct.unpack_from(f"<{nt}I", buf, off)); off += 4 * nt
    rcut, rcut_smth = struct.unpack_from("<dd", buf, off); off += 16
    emb = list(struct.unpack_from("<3I", buf, off)); off += 12
    (axis,) = struct.unpack_from("<I", buf, off); off += 4
    fit = list(struct.unpack_from("<3I", buf, off)); off += 12
    (prec,) = struct.unpack_from("<I", buf, off); off += 4
    type_map = []
    for _ in range(nt):
        type_map.append(buf[off:off + 16].split(b"\0")[0].decode()); off += 16

    def take(n, shape):
        nonlocal off
        a = np.frombuffer(buf, dtype="<f8", count=n, offset=off).reshape(shape).copy()
        off += 8 * n
        return a
    davg = take(nt * nt * 4, (nt, nt, 4))
    dstd = take(nt * nt * 4, (nt, nt, 4))
    eb, fb = emb_block_size(emb), fit_block_size(emb, axis, fit)
    emb_params = take(nt * nt * eb, (nt * nt, eb))
    fit_params = take(nt * fb, (nt, fb))
    bias = take(nt, (nt,))
    return dict(type_map=type_map, sel=sel, rcut=rcut, rcut_smth=rcut_smth, emb=emb, axis=axis,
                fit=fit, davg=davg, dstd=dstd, emb_params=emb_params, fit_params=fit_params,
                bias_atom_e=bias, precision="mixed" if prec == 1 else "fp64")


def read_model(path: str) -> dict:
    with open(path, "rb") as f:
        return from_bytes(f.read())
