"""DPA4C-Nano model files: layout constants, seeded random initialisation,
writer and reader.

DPA4C is the reference's compressed degree-wise descriptor
(dpa4c-runtime/include/dpa_chain/graph_compress.cuh,
deepmd-op/overlays/op/pt/dpa4c/graph_compress_kernel.cuh:78-760). Its
production profile is "Nano": 8 scalar channels, angular degrees up to 2, no
spin branch, no radial modes, a 70-wide descriptor and a fitting net of one
70 -> 96 hidden layer plus a linear head
(deepmd-op/overlays/op/pt/graph_fitting.cu:333-341). The widths follow the
reference's profile arithmetic (graph_compress_launch.h:103-126, 262-327):

    C0 = 8 scalar channels, C1 = 4 degree-one channels, C2 = 4 degree-two
    channels, K1 = C2 = 4 degree-one probes, K2 = 2 degree-two probes;
    moments  [C0 scalar][3 x C1 vector][5 x C2 tensor]       = 40
    output   [C0 scalar][Gram1 10][Gram2 10][Bis112 20][Bis222 4]
             [Quartic 8][2 divisors][C0 type embedding]       = 70

File layout (little endian), read by the C++ loader in csrc/model.cpp:

    8 bytes   magic "DPAMDC4N"
    u32       version (1)
    u32       ntypes
    u32[nt]   sel: neighbour capacity per type of the standalone neighbour
              list (an overflow is an error, never a truncation)
    f64       rcut, eps, degree_floor, table_stride
    u32       interval_count, channels (8), lmax (2)
    u32       n_layer, u32[n_layer] hidden widths, u32 activation (0 tanh,
              1 silu), u32 resnet mask (bit l: identity residual on square
              layer l)
    char[nt][16] type_map, NUL padded
    f32[interval_count][6][C0]  radial table: coefficient k of channel c of
              interval i at [i][k][c]; radial_c(r) = sum_k coef_k x^k with
              x = r - i * table_stride
    f32[nt*nt][C0][2]  PairFiLM (scale, shift) of pair (ti, tj) at ti*nt+tj
    f32[C1][C1] vector alignment, f32[C2][C2] tensor alignment,
    f32[C1][K1] vector probes,    f32[C2][K2] tensor probes
    f32[nt][C0] type embedding
    f32[70] output mean, f32[70] output inverse standard deviation
    f32 per layer W[in][out], b[out]; f32[H] head weights; f32 head bias
    f64[nt]   bias_atom_e
"""
from __future__ import annotations

import struct

import numpy as np

from .systems import Stream

MAGIC = b"DPAMDC4N"

C0, LMAX = 8, 2
C1, C2 = 4, 4
K1, K2 = C2, 2
N_MOMENT = C0 + 3 * C1 + 5 * C2
GRAM1 = C1 * (C1 + 1) // 2
GRAM2 = C2 * (C2 + 1) // 2
BIS112 = K1 * (K1 + 1) // 2 * K2
BIS222 = 4
QUARTIC = K1 * K2
OUT_SCALAR = 0
OUT_GRAM1 = C0
OUT_GRAM2 = OUT_GRAM1 + GRAM1
OUT_BIS112 = OUT_GRAM2 + GRAM2
OUT_BIS222 = OUT_BIS112 + BIS112
OUT_QUARTIC = OUT_BIS222 + BIS222
OUT_DIVISOR = OUT_QUARTIC + QUARTIC
OUT_TYPE = OUT_DIVISOR + 2
OUT_WIDTH = OUT_TYPE + C0
assert OUT_WIDTH == 70

ACT_TANH, ACT_SILU = 0, 1

KINDS = {
    "cu": dict(type_map=["Cu"], sel=[128]),
    "water": dict(type_map=["O", "H"], sel=[64, 128]),
    "hea": dict(type_map=["Co", "Cr", "Fe", "Ni"], sel=[48, 48, 48, 48]),
    "cuni": dict(type_map=["Cu", "Ni"], sel=[80, 80]),
}


def quintic_hermite(h, f0, d0, s0, f1, d1, s1):
    """Coefficients a0..a5 of p(x) on [0, h] with p, p', p'' equal to
    (f0, d0, s0) at x = 0 and (f1, d1, s1) at x = h (arrays broadcast)."""
    a0, a1, a2 = f0, d0, 0.5 * s0
    # remaining cubic part q(x) = a3 x^3 + a4 x^4 + a5 x^5 fixes the far end
    r0 = f1 - (a0 + a1 * h + a2 * h * h)
    r1 = d1 - (a1 + 2 * a2 * h)
    r2 = s1 - 2 * a2
    A = np.array([[h ** 3, h ** 4, h ** 5],
                  [3 * h ** 2, 4 * h ** 3, 5 * h ** 4],
                  [6 * h, 12 * h ** 2, 20 * h ** 3]])
    rhs = np.stack([r0, r1, r2], axis=0)
    sol = np.linalg.solve(A, rhs.reshape(3, -1)).reshape(rhs.shape)
    return np.stack([a0, a1, a2, sol[0], sol[1], sol[2]], axis=0)


def radial_table(st: Stream, rcut: float, stride: float, channels: int, nbasis: int = 6,
                 dtype=np.float32):
    """C2 quintic spline table of smooth random radial functions.

    radial_c(r) = sum_k alpha_ck exp(-(r - mu_k)^2 / (2 sigma^2)) with mu_k
    evenly spaced over [0, rcut]; each interval is the quintic Hermite
    interpolant of value, slope and curvature at its two knots, so the table
    is C2 across knots (to the rounding of the stored coefficients). Returns
    ([intervals][6][channels] of dtype, intervals)."""
    n_int = int(np.ceil(rcut / stride - 1e-9)) + 1
    knots = np.arange(n_int + 1) * stride
    mu = np.linspace(0.0, rcut, nbasis)
    sig = rcut / (nbasis - 1)
    alpha = st.normal(channels * nbasis).reshape(channels, nbasis)
    z = (knots[:, None] - mu[None, :]) / sig
    g = np.exp(-0.5 * z * z)
    dg = -z / sig * g
    ddg = (z * z - 1.0) / (sig * sig) * g
    f = g @ alpha.T        # [knots][channels]
    d = dg @ alpha.T
    s = ddg @ alpha.T
    coef = quintic_hermite(stride, f[:-1], d[:-1], s[:-1], f[1:], d[1:], s[1:])  # [6][int][ch]
    return np.ascontiguousarray(coef.transpose(1, 0, 2)).astype(dtype), n_int


def random_model(kind: str, seed: int, **overrides) -> dict:
    """Seeded random DPA4C-Nano model. rcut 6 A (the reference's production
    cutoff, dpa4c-runtime/config/engine.production.json.in:17), eps 1e-3 A,
    degree floor 1e-2, table stride 0.02 A; fitting [96] tanh."""
    spec = dict(KINDS[kind])
    spec.update(dict(rcut=6.0, eps=1e-3, degree_floor=1e-2, table_stride=0.02, fit=[96],
                     act=ACT_TANH, resnet=0))
    spec.update(overrides)
    nt = len(spec["type_map"])
    st = Stream(seed, 11)
    table, n_int = radial_table(st, spec["rcut"], spec["table_stride"], C0)
    film = np.empty((nt * nt, C0, 2))
    film[..., 0] = 1.0 + 0.3 * st.normal(nt * nt * C0).reshape(nt * nt, C0)
    film[..., 1] = 0.2 * st.normal(nt * nt * C0).reshape(nt * nt, C0)
    Ma = np.eye(C1) + 0.3 * st.normal(C1 * C1).reshape(C1, C1)
    Mt = np.eye(C2) + 0.3 * st.normal(C2 * C2).reshape(C2, C2)
    Pv = st.normal(C1 * K1).reshape(C1, K1) / np.sqrt(C1)
    Pt = st.normal(C2 * K2).reshape(C2, K2) / np.sqrt(C2)
    temb = st.normal(nt * C0).reshape(nt, C0)
    mean = 0.1 * st.normal(OUT_WIDTH)
    inv_std = 1.0 / (0.5 + 0.5 * np.abs(st.normal(OUT_WIDTH)))
    layers = []
    din = OUT_WIDTH
    for w in spec["fit"]:
        W = st.normal(din * w).reshape(din, w) / np.sqrt(din + w)
        b = 0.1 * st.normal(w)
        layers.append((W, b))
        din = w
    w_head = st.normal(din) / np.sqrt(din + 1)
    b_head = float(st.normal(1)[0])
    bias = st.normal(nt)
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
    return dict(type_map=list(spec["type_map"]), sel=list(spec["sel"]), rcut=float(spec["rcut"]),
                eps=float(spec["eps"]), degree_floor=float(spec["degree_floor"]),
                table_stride=float(spec["table_stride"]), interval_count=n_int, channels=C0,
                lmax=LMAX, fit=list(spec["fit"]), act=int(spec["act"]), resnet=int(spec["resnet"]),
                table=table, film=f32(film), Ma=f32(Ma), Mt=f32(Mt), Pv=f32(Pv), Pt=f32(Pt),
                type_embedding=f32(temb), out_mean=f32(mean), out_inv_std=f32(inv_std),
                layers=[(f32(W), f32(b)) for W, b in layers], w_head=f32(w_head),
                b_head=np.float32(b_head), bias_atom_e=np.asarray(bias, np.float64))


def to_bytes(m: dict) -> bytes:
    nt = len(m["type_map"])
    out = [MAGIC, struct.pack("<II", 1, nt), struct.pack(f"<{nt}I", *m["sel"]),
           struct.pack("<4d", m["rcut"], m["eps"], m["degree_floor"], m["table_stride"]),
           struct.pack("<3I", m["interval_count"], m["channels"], m["lmax"]),
           struct.pack("<I", len(m["fit"])), struct.pack(f"<{len(m['fit'])}I", *m["fit"]),
           struct.pack("<II", m["act"], m["resnet"])]
    for name in m["type_map"]:
        b = name.encode()[:15]
        out.append(b + b"\0" * (16 - len(b)))
    f32 = lambda a: np.ascontiguousarray(a, dtype="<f4").tobytes()  # noqa: E731
    for key in ("table", "film", "Ma", "Mt", "Pv", "Pt", "type_embedding", "out_mean",
                "out_inv_std"):
        out.append(f32(m[key]))
    for W, b in m["layers"]:
        out += [f32(W), f32(b)]
    out += [f32(m["w_head"]), f32(np.array([m["b_head"]]))]
    out.append(np.ascontiguousarray(m["bias_atom_e"], dtype="<f8").tobytes())
    return b"".join(out)


def from_bytes(buf: bytes) -> dict:
    if buf[:8] != MAGIC:
        raise ValueError("not a DPAMDC4N model file")
    off = 8
    ver, nt = struct.unpack_from("<II", buf, off); off += 8
    if ver != 1:
        raise ValueError(f"unsupported model version {ver}")
    sel = list(struct.unpack_from(f"<{nt}I", buf, off)); off += 4 * nt
    rcut, eps, floor, stride = struct.unpack_from("<4d", buf, off); off += 32
    n_int, ch, lmax = struct.unpack_from("<3I", buf, off); off += 12
    (nl,) = struct.unpack_from("<I", buf, off); off += 4
    fit = list(struct.unpack_from(f"<{nl}I", buf, off)); off += 4 * nl
    act, resnet = struct.unpack_from("<II", buf, off); off += 8
    if ch != C0 or lmax != LMAX:
        raise ValueError(f"only the Nano profile (channels {C0}, lmax {LMAX}) is supported")
    type_map = []
    for _ in range(nt):
        type_map.append(buf[off:off + 16].split(b"\0")[0].decode()); off += 16

    def take(shape, dt="<f4"):
        nonlocal off
        n = int(np.prod(shape))
        a = np.frombuffer(buf, dtype=dt, count=n, offset=off).reshape(shape).copy()
        off += np.dtype(dt).itemsize * n
        return a
    m = dict(type_map=type_map, sel=sel, rcut=rcut, eps=eps, degree_floor=floor,
             table_stride=stride, interval_count=n_int, channels=ch, lmax=lmax, fit=fit, act=act,
             resnet=resnet)
    m["table"] = take((n_int, 6, C0))
    m["film"] = take((nt * nt, C0, 2))
    m["Ma"], m["Mt"] = take((C1, C1)), take((C2, C2))
    m["Pv"], m["Pt"] = take((C1, K1)), take((C2, K2))
    m["type_embedding"] = take((nt, C0))
    m["out_mean"], m["out_inv_std"] = take((OUT_WIDTH,)), take((OUT_WIDTH,))
    layers, din = [], OUT_WIDTH
    for w in fit:
        layers.append((take((din, w)), take((w,))))
        din = w
    m["layers"] = layers
    m["w_head"] = take((din,))
    m["b_head"] = np.float32(take((1,))[0])
    m["bias_atom_e"] = take((nt,), "<f8")
    if off != len(buf):
        raise ValueError("trailing bytes in DPAMDC4N model file")
    return m


def write_model(path: str, m: dict) -> str:
    with open(path, "wb") as f:
        f.write(to_bytes(m))
    return path
