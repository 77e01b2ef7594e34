"""MI355X-native DeePMD se_e2_a energy / force / virial evaluation.

Python front end over the C ABI of libdpamd.so (include/dp_amd.h). `DeepPot`
mirrors the reference's C++ model API (deepmd-op/overlays/api_cc/include/DeepPot.h:451-926):
init(model, gpu_rank, file_content), compute(...) with and without a LAMMPS
neighbour list, cutoff(), numb_types(), dim_fparam(), dim_aparam(),
get_type_map(). Errors raise DeepmdException, as the reference raises
deepmd::deepmd_exception (DeepPotPTExpt.cc:295-309).

The library must be built (`make -C csrc`, or __graft_entry__.build()); there
is no CPU fallback: without the HIP library every compute call fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import dpa4c, model, systems  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdpamd.so")
_LIB = None

MAX_TYPES = 8
STAGE_NLIST, STAGE_EXT_COORD, STAGE_MAPPING, STAGE_DESCRPT = 0, 1, 2, 3
STAGE_ATOM_ENERGY, STAGE_EDGE_GRAD, STAGE_DEDD, STAGE_EXT_TYPE = 4, 5, 6, 7
STAGE_C4_MOMENTS, STAGE_C4_COTANGENTS = 8, 9
PREC_FP64, PREC_MIXED, PREC_MODEL = 0, 1, -1
MODEL_SE_E2_A, MODEL_DPA4C = 0, 1

EXPORTED = ("dp_create", "dp_destroy", "dp_get_info", "dp_last_error", "dp_compute",
            "dp_compute_nlist", "dp_compute_device", "dp_compute_device_async",
            "dp_compute_device_noalloc", "dp_sync",
            "dp_graph_stats", "dp_compute_canonical_graph_device", "dp_compute_edges_device",
            "dp_compute_edges_device_f32",
            "dp_debug_copy", "dp_debug_keep", "dp_debug_fused_rows", "dp_stage_times",
            "dp_device_bytes")


class DeepmdException(RuntimeError):
    """Raised for every failure reported through the C ABI."""


class ModelInfo(C.Structure):
    _fields_ = [("ntypes", C.c_int), ("nnei", C.c_int), ("sel", C.c_int * MAX_TYPES),
                ("rcut", C.c_double), ("rcut_smth", C.c_double), ("emb", C.c_int * 3),
                ("axis", C.c_int), ("fit", C.c_int * 3), ("dim_fparam", C.c_int),
                ("dim_aparam", C.c_int), ("precision", C.c_int),
                ("type_map", (C.c_char * 16) * MAX_TYPES), ("model_kind", C.c_int)]


def lib():
    """Load libdpamd.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise DeepmdException(f"{LIB_PATH} not built: run `make -C {os.path.join(_HERE, 'csrc')}`")
        L = C.CDLL(LIB_PATH)
        P, I, D = C.c_void_p, C.c_int, C.c_double
        L.dp_create.argtypes = [C.c_char_p, I, P, C.c_size_t, I, C.POINTER(P)]
        L.dp_destroy.argtypes = [P]
        L.dp_destroy.restype = None
        L.dp_get_info.argtypes = [P, C.POINTER(ModelInfo)]
        L.dp_last_error.argtypes = [P]
        L.dp_last_error.restype = C.c_char_p
        L.dp_compute.argtypes = [P, I, P, P, P, P, P, P, P, P]
        L.dp_compute_nlist.argtypes = [P, I, I, P, P, P, I, P, P, P, I, I, P, P, P, P, P]
        L.dp_compute_device.argtypes = [P, I, P, P, P, I, P, P, P, P, P, P]
        L.dp_compute_device_async.argtypes = [P, I, P, P, P, I, P, P, P, P, P, P]
        L.dp_compute_device_noalloc.argtypes = [P, I, P, P, P, P, P, P, P, P, P]
        L.dp_sync.argtypes = [P]
        L.dp_graph_stats.argtypes = [P, C.POINTER(C.c_long), C.POINTER(C.c_long)]
        L.dp_compute_canonical_graph_device.argtypes = [P, P, P, P, P, P, P, P, P, P, I, I,
                                                        C.c_int64, P]
        L.dp_compute_edges_device.argtypes = [P, P, P, P, P, P, P, P, I, I, I, P]
        L.dp_compute_edges_device_f32.argtypes = [P, P, P, P, P, P, P, P, I, I, I, P]
        L.dp_debug_copy.argtypes = [P, I, P, C.c_size_t]
        L.dp_debug_copy.restype = C.c_long
        L.dp_debug_keep.argtypes = [P, I]
        L.dp_debug_fused_rows.argtypes = [P, I]
        L.dp_stage_times.argtypes = [P, I, P, I, P, C.c_size_t]
        L.dp_device_bytes.argtypes = [P]
        L.dp_device_bytes.restype = C.c_size_t
        _ = D
        _LIB = L
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class DeepPot:
    """A DeePMD model (se_e2_a, or DPA4C-Nano) evaluated on one gfx950 GPU;
    the family is read from the model file."""

    def __init__(self, model_path: str | None = None, gpu_rank: int = 0,
                 file_content: bytes | None = None, precision: int = PREC_MODEL):
        self._h = None
        if model_path is not None or file_content is not None:
            self.init(model_path, gpu_rank, file_content, precision)

    def init(self, model_path, gpu_rank=0, file_content=None, precision=PREC_MODEL):
        L = lib()
        h = C.c_void_p()
        buf = file_content if file_content else None
        rc = L.dp_create(model_path.encode() if model_path else None, gpu_rank,
                         buf, len(buf) if buf else 0, precision, C.byref(h))
        if rc != 0:
            msg = L.dp_last_error(h).decode() if h else "dp_create failed"
            if h:
                L.dp_destroy(h)
            raise DeepmdException(f"dp_create failed ({rc}): {msg}")
        self._h = h
        info = ModelInfo()
        L.dp_get_info(h, C.byref(info))
        self.info = info
        self._ntypes = info.ntypes
        self.nnei = info.nnei
        self.sel = [info.sel[t] for t in range(info.ntypes)]
        self.model_kind = info.model_kind
        self.ndescrpt = 70 if info.model_kind == MODEL_DPA4C else info.emb[2] * info.axis

    def __del__(self):
        if getattr(self, "_h", None):
            lib().dp_destroy(self._h)
            self._h = None

    def _check(self, rc):
        if rc != 0:
            raise DeepmdException(f"({rc}) {lib().dp_last_error(self._h).decode()}")

    # ---- metadata (DeepPotPTExpt.h:103-154) ------------------------------
    def cutoff(self) -> float:
        return self.info.rcut

    def numb_types(self) -> int:
        return self._ntypes

    def numb_types_spin(self) -> int:
        return 0

    def dim_fparam(self) -> int:
        return self.info.dim_fparam

    def dim_aparam(self) -> int:
        return self.info.dim_aparam

    def get_type_map(self) -> str:
        return " ".join(self.info.type_map[t].value.decode() for t in range(self._ntypes))

    # ---- evaluation --------------------------------------------------------
    def compute(self, coord, atype, box=None, atomic=False):
        """Standalone evaluation; returns (energy, force[n,3], virial[9]) and, when
        atomic, also atom_energy[n], atom_virial[n,9]."""
        coord = np.ascontiguousarray(coord, np.float64).reshape(-1, 3)
        atype = np.ascontiguousarray(atype, np.int32).reshape(-1)
        n = len(atype)
        if coord.shape[0] != n:
            raise DeepmdException("coord and atype sizes differ")
        boxa = None if box is None else np.ascontiguousarray(box, np.float64).reshape(9)
        e = C.c_double()
        f = np.zeros((n, 3))
        v = np.zeros(9)
        ae = np.zeros(n) if atomic else None
        av = np.zeros((n, 9)) if atomic else None
        self._check(lib().dp_compute(self._h, n, _ptr(coord), _ptr(atype), _ptr(boxa), C.byref(e),
                                     _ptr(f), _ptr(v), _ptr(ae), _ptr(av)))
        if atomic:
            return e.value, f, v, ae, av
        return e.value, f, v

    def compute_nlist(self, coord, atype, box, nghost, ilist, numneigh, firstneigh, ago=0,
                      atomic=False, neigh_mask=0):
        """LAMMPS-path evaluation over nall = nloc + nghost atoms; `firstneigh` is a
        list of int arrays (one per ilist entry). Forces cover all nall atoms."""
        coord = np.ascontiguousarray(coord, np.float64).reshape(-1, 3)
        atype = np.ascontiguousarray(atype, np.int32).reshape(-1)
        nall = len(atype)
        ilist = np.ascontiguousarray(ilist, np.int32)
        numneigh = np.ascontiguousarray(numneigh, np.int32)
        rows = [np.ascontiguousarray(r, np.int32) for r in firstneigh]
        ptrs = (C.c_void_p * max(len(rows), 1))(*[r.ctypes.data for r in rows])
        boxa = None if box is None else np.ascontiguousarray(box, np.float64).reshape(9)
        e = C.c_double()
        f = np.zeros((nall, 3))
        v = np.zeros(9)
        ae = np.zeros(nall) if atomic else None
        av = np.zeros((nall, 9)) if atomic else None
        self._check(lib().dp_compute_nlist(self._h, nall, nghost, _ptr(coord), _ptr(atype),
                                           _ptr(boxa), len(ilist), _ptr(ilist), _ptr(numneigh),
                                           C.cast(ptrs, C.c_void_p), neigh_mask, ago, C.byref(e),
                                           _ptr(f), _ptr(v), _ptr(ae), _ptr(av)))
        if atomic:
            return e.value, f, v, ae, av
        return e.value, f, v

    def compute_device(self, d_coord: int, d_atype: int, natoms: int, box, d_energy: int,
                       d_force: int, d_virial: int, d_atom_energy: int = 0,
                       d_atom_virial: int = 0, ago: int = 0, stream: int = 0):
        """Device-resident evaluation on raw device pointers (ints)."""
        boxa = np.ascontiguousarray(box, np.float64).reshape(9)
        self._check(lib().dp_compute_device(self._h, natoms, d_coord, d_atype, _ptr(boxa), ago,
                                            d_energy, d_force, d_virial, d_atom_energy or None,
                                            d_atom_virial or None, stream or None))

    def compute_device_noalloc(self, d_coord: int, d_atype: int, natoms: int, box,
                               d_energy: int, d_force: int, d_virial: int,
                               d_atom_energy: int = 0, d_atom_virial: int = 0, stream: int = 0):
        """dp_compute_device_noalloc: the device-resident evaluation with
        every work buffer in the library's static per-GPU scratch."""
        boxa = np.ascontiguousarray(box, np.float64).reshape(9)
        self._check(lib().dp_compute_device_noalloc(self._h, natoms, d_coord, d_atype,
                                                    _ptr(boxa), d_energy, d_force, d_virial,
                                                    d_atom_energy or None, d_atom_virial or None,
                                                    stream or None))

    def compute_device_async(self, d_coord: int, d_atype: int, natoms: int, box, d_energy: int,
                             d_force: int, d_virial: int, d_atom_energy: int = 0,
                             d_atom_virial: int = 0, ago: int = 1, stream: int = 0):
        """Enqueue a device-resident evaluation and return without waiting
        (dp_compute_device_async); sync() waits and reports deferred errors."""
        boxa = np.ascontiguousarray(box, np.float64).reshape(9)
        self._check(lib().dp_compute_device_async(self._h, natoms, d_coord, d_atype, _ptr(boxa),
                                                  ago, d_energy, d_force, d_virial,
                                                  d_atom_energy or None, d_atom_virial or None,
                                                  stream or None))

    def compute_canonical_graph_device(self, d_atom_energy: int, d_force: int,
                                       d_atom_virial: int, d_atype: int, d_source: int,
                                       d_edge_vec: int, d_destination_row_ptr: int,
                                       d_source_row_ptr: int, d_source_order: int, nloc: int,
                                       nall_nodes: int, edge_storage: int, stream: int = 0):
        """DPA4C evaluation of a compact canonical graph on raw device pointers
        (dp_compute_canonical_graph_device, mirroring
        DeepPot::compute_canonical_graph_gpu)."""
        self._check(lib().dp_compute_canonical_graph_device(
            self._h, d_atom_energy or None, d_force, d_atom_virial, d_atype, d_source, d_edge_vec,
            d_destination_row_ptr, d_source_row_ptr, d_source_order, nloc, nall_nodes,
            edge_storage, stream or None))

    def compute_edges_device(self, d_atom_energy: int, d_force: int, d_atom_virial: int,
                             d_coord: int, d_atype: int, d_edge_index: int, d_edge_vec: int,
                             nloc: int, nedge: int, nall_nodes: int = 0, fp32: bool = False,
                             stream: int = 0):
        """Evaluation of a device edge graph on raw device pointers
        (dp_compute_edges_device[_f32], mirroring DeepPot::compute_edges_gpu)."""
        f = lib().dp_compute_edges_device_f32 if fp32 else lib().dp_compute_edges_device
        self._check(f(self._h, d_atom_energy or None, d_force, d_atom_virial, d_coord or None,
                      d_atype, d_edge_index or None, d_edge_vec or None, nloc, nedge, nall_nodes,
                      stream or None))

    def sync(self):
        """Wait for the queued asynchronous evaluations (dp_sync)."""
        self._check(lib().dp_sync(self._h))

    def graph_stats(self):
        """(graphs in use, captures, replays) of the DPAMD_GRAPH replay."""
        cap, rep = C.c_long(0), C.c_long(0)
        on = lib().dp_graph_stats(self._h, C.byref(cap), C.byref(rep))
        return bool(on == 1), cap.value, rep.value

    # ---- introspection -----------------------------------------------------
    def stage(self, which: int, dtype, shape):
        n = lib().dp_debug_copy(self._h, which, None, 0)
        if n < 0:
            self._check(int(n))
        out = np.zeros(shape, dtype=dtype)
        assert out.nbytes == n, (out.nbytes, n)
        got = lib().dp_debug_copy(self._h, which, _ptr(out), out.nbytes)
        if got < 0:
            self._check(int(got))
        return out

    def keep_stages(self, on=True):
        """Store the per-slot edge gradients of the evaluations that follow, so
        stage(STAGE_EDGE_GRAD) can return them (dp_debug_keep)."""
        self._check(lib().dp_debug_keep(self._h, 1 if on else 0))

    def set_fused_rows(self, rows):
        """fp64 se_e2_a: use the fused dE/dD -> dE/dT kernel when every atom
        type has at least `rows` atoms (0: always; dp_debug_fused_rows)."""
        self._check(lib().dp_debug_fused_rows(self._h, int(rows)))

    def enable_stage_timing(self, on=True):
        times = (C.c_double * 16)()
        lib().dp_stage_times(self._h, 1 if on else 0, times, 16, None, 0)

    def stage_times(self):
        times = (C.c_double * 16)()
        names = C.create_string_buffer(512)
        n = lib().dp_stage_times(self._h, 1, times, 16, names, 512)
        labels = names.raw.split(b"\0")[:n]
        return {labels[q].decode(): times[q] for q in range(n)}

    def device_bytes(self) -> int:
        return int(lib().dp_device_bytes(self._h))
