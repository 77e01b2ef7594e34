"""Native pieces that need no GPU: the C ABI library loads and exports every
symbol include/dp_amd.h declares, fails cleanly without a GPU or with a bad
model, the C++ façade compiles and links, the device tanh (host build) is
accurate, and the oracle is clean under ASan/UBSan."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from _pkg import PKG_DIR, ROOT

HEADER = os.path.join(ROOT, "include", "dp_amd.h")


def declared_symbols():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|long|size_t|const char\*)\s+(dp_\w+)\(", txt, re.M)))


def test_library_exports_declared_symbols(dp):
    syms = declared_symbols()
    assert len(syms) >= 10
    L = dp.lib()
    for s in syms:
        assert hasattr(L, s), f"{s} not exported by libdpamd.so"
    assert set(syms) == set(dp.EXPORTED)


def test_library_links_no_vendor_blas(dp):
    """Every product on the path is this library's own kernel: the shared
    library needs no BLAS / GEMM library (rocBLAS, hipBLAS, hipBLASLt)."""
    import subprocess
    lib_path = dp.lib()._name
    out = subprocess.run(["readelf", "-d", lib_path], capture_output=True, text=True, check=True).stdout
    needed = [ln for ln in out.splitlines() if "(NEEDED)" in ln]
    assert needed, out
    assert not [ln for ln in needed if "blas" in ln.lower()], needed


def test_bad_model_is_reported(dp):
    L = dp.lib()
    h = ctypes.c_void_p()
    junk = b"NOTAMODEL" * 10
    rc = L.dp_create(None, 0, junk, len(junk), 0, ctypes.byref(h))
    assert rc == -2
    assert b"DPAMDSEA" in L.dp_last_error(h)
    L.dp_destroy(h)
    with pytest.raises(dp.DeepmdException):
        dp.DeepPot(file_content=junk)


def test_model_precision_field(dp):
    """The model file records the precision it is evaluated in (the header
    word after the fitting widths): the Python writer and reader round-trip
    it, files written before the word was used read as fp64, and the C
    loader rejects a value other than 0 or 1 before it looks for a GPU."""
    import struct
    m = dp.model.random_model("water", seed=3)
    assert dp.model.from_bytes(dp.model.to_bytes(m))["precision"] == "fp64"
    m["precision"] = "mixed"
    b = dp.model.to_bytes(m)
    assert dp.model.from_bytes(b)["precision"] == "mixed"
    nt = len(m["type_map"])
    off = 8 + 8 + 4 * nt + 16 + 12 + 4 + 12  # magic, version/ntypes, sel, rcut, emb, axis, fit
    assert struct.unpack_from("<I", b, off)[0] == 1
    bad = bytearray(b)
    struct.pack_into("<I", bad, off, 2)
    L = dp.lib()
    h = ctypes.c_void_p()
    rc = L.dp_create(None, 0, bytes(bad), len(bad), -1, ctypes.byref(h))
    assert rc == -2 and b"precision field" in L.dp_last_error(h)
    L.dp_destroy(h)
    h = ctypes.c_void_p()
    rc = L.dp_create(None, 0, b, len(b), 7, ctypes.byref(h))
    assert rc == -1 and b"DP_PREC_MODEL" in L.dp_last_error(h)
    L.dp_destroy(h)


def test_unsupported_shape_is_reported(dp):
    m = dp.model.random_model("water", seed=1, emb=[8, 16, 32])
    with pytest.raises(dp.DeepmdException, match="not compiled"):
        dp.DeepPot(file_content=dp.model.to_bytes(m))


def _gpu_visible(dp):
    import importlib
    hip = importlib.import_module("dpamd.hip")
    try:
        return hip.device_count() > 0
    except Exception:
        return False


def test_no_gpu_fails_loudly(dp):
    if _gpu_visible(dp):
        pytest.skip("a GPU is visible")
    mb = dp.model.to_bytes(dp.model.random_model("water", seed=1))
    with pytest.raises(dp.DeepmdException, match="HIP device|gfx950"):
        dp.DeepPot(file_content=mb)


def test_tanh_fast_accuracy(tmp_path):
    exe = tmp_path / "tanh_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "native", "tanh_check.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_embedding_layouts_agree(tmp_path):
    """Host packing layout == the kernels' compile-time layout (fp64 and fp32)."""
    exe = tmp_path / "layout_check"
    subprocess.run(["g++", "-O1", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "native", "layout_check.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def build_facade(tmp_path):
    exe = tmp_path / "facade_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "native", "facade_check.cpp"), "-o", str(exe),
                    "-L", PKG_DIR, "-ldpamd", f"-Wl,-rpath,{PKG_DIR}"], check=True)
    return exe


def build_pair_shape(tmp_path):
    """The pair-style member check, compiled the way the reference plugin is
    (LMPPLUGIN: headers found by their bare names on the include path)."""
    exe = tmp_path / "pair_shape_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror",
                    "-I", os.path.join(ROOT, "include", "deepmd_amd"),
                    os.path.join(ROOT, "tests", "native", "pair_shape_check.cpp"), "-o", str(exe),
                    "-L", PKG_DIR, "-ldpamd", f"-Wl,-rpath,{PKG_DIR}"], check=True)
    return exe


def build_backend_shape(tmp_path):
    """The backend adapter hosted under the reference's backend interface
    (tests/native/backend_shape_check.cpp), compiled with every warning an
    error."""
    exe = tmp_path / "backend_shape_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Woverloaded-virtual",
                    "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "native", "backend_shape_check.cpp"), "-o",
                    str(exe), "-L", PKG_DIR, "-ldpamd", f"-Wl,-rpath,{PKG_DIR}"], check=True)
    return exe


def test_backend_adapter_implements_the_backend_interface(tmp_path):
    """DeepPotBackendAMD implements every pure virtual of the reference's
    deepmd::DeepPotBackend with matching signatures: the class declared as a
    maintainer would declare it compiles and can be constructed."""
    exe = build_backend_shape(tmp_path)
    r = subprocess.run([str(exe), "shape"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "SHAPE ok" in r.stdout, r.stdout + r.stderr


def test_pair_style_members_compile_and_deviation_statistics(tmp_path):
    """The façade hosts pair_base.h / pair_deepmd.h's model members (the
    translation unit compiles only if every bound type and called method
    exists) and the model-deviation statistics match their closed forms."""
    exe = build_pair_shape(tmp_path)
    r = subprocess.run([str(exe), "stats"], capture_output=True, text=True)
    assert r.returncode == 0 and "STATS OK" in r.stdout, r.stdout + r.stderr


def write_input(path, coord, atype, box):
    with open(path, "wb") as f:
        f.write(np.int32(len(atype)).tobytes())
        f.write(np.ascontiguousarray(coord, np.float64).tobytes())
        f.write(np.ascontiguousarray(atype, np.int32).tobytes())
        f.write(np.ascontiguousarray(box, np.float64).tobytes())


def test_facade_builds_and_throws_without_gpu(dp, tmp_path):
    exe = build_facade(tmp_path)
    if _gpu_visible(dp):
        pytest.skip("a GPU is visible (the GPU test runs the façade)")
    mpath = tmp_path / "m.dp"
    dp.model.write_model(str(mpath), dp.model.random_model("water", seed=1))
    coord, atype, box = dp.systems.build(0)
    write_input(tmp_path / "in.bin", coord, atype, box)
    r = subprocess.run([str(exe), str(mpath), str(tmp_path / "in.bin")], capture_output=True, text=True)
    assert r.returncode == 3 and "EXC" in r.stdout


def test_oracle_sanitizers(dp, tmp_path):
    """Build the oracle with ASan + UBSan and evaluate the 192-atom water box."""
    src = os.path.join(ROOT, "oracle")
    drv = tmp_path / "drv.c"
    drv.write_text(r'''
#include <stdio.h>
#include <stdlib.h>
#include "se_e2_a.h"
int main(int argc, char** argv) {
  FILE* f = fopen(argv[1], "rb"); int n, nt, sel[8], emb[3], fit[3], axis; double rc, rs;
  if (fread(&n, 4, 1, f) != 1) return 2;
  double* coord = malloc(24 * n); int* at = malloc(4 * n); double box[9];
  fread(coord, 8, 3 * n, f); fread(at, 4, n, f); fread(box, 8, 9, f);
  fread(&nt, 4, 1, f); fread(sel, 4, nt, f); fread(&rc, 8, 1, f); fread(&rs, 8, 1, f);
  fread(emb, 4, 3, f); fread(&axis, 4, 1, f); fread(fit, 4, 3, f);
  long nd, ne, nf; fread(&nd, 8, 1, f); fread(&ne, 8, 1, f); fread(&nf, 8, 1, f);
  double* davg = malloc(8 * nd); double* dstd = malloc(8 * nd); double* ep = malloc(8 * ne);
  double* fp = malloc(8 * nf); double bias[8];
  fread(davg, 8, nd, f); fread(dstd, 8, nd, f); fread(ep, 8, ne, f); fread(fp, 8, nf, f);
  fread(bias, 8, nt, f); fclose(f);
  orc_model m = {0}; m.ntypes = nt; int acc = 0;
  for (int t = 0; t < nt; ++t) { m.sel[t] = sel[t]; m.sec[t] = acc; acc += sel[t]; }
  m.sec[nt] = acc; m.nnei = acc; m.rcut = rc; m.rcut_smth = rs; m.axis = axis;
  for (int k = 0; k < 3; ++k) { m.emb[k] = emb[k]; m.fit[k] = fit[k]; }
  m.davg = davg; m.dstd = dstd; m.emb_params = ep; m.fit_params = fp; m.bias_atom_e = bias;
  int nall = orc_ghost_count(n, coord, box, rc);
  double* ext = malloc(24 * nall); int* et = malloc(4 * nall); int* mp = malloc(4 * nall);
  orc_build_ghosts(n, coord, at, box, rc, nall, ext, et, mp);
  long* off = malloc(8 * (n + 1));
  long nc = orc_candidates_cell(n, nall, ext, et, NULL, rc, 0, off, NULL);
  int* cand = malloc(4 * (nc + 1));
  orc_candidates_cell(n, nall, ext, et, NULL, rc, nc, off, cand);
  int* nl = malloc(4 * n * m.nnei);
  orc_format_nlist(&m, n, ext, et, off, cand, nl);
  double* ae = malloc(8 * n); double* frc = malloc(24 * nall); double v[9];
  double* av = malloc(72 * nall);
  orc_eval(&m, n, nall, ext, et, nl, 1, ae, NULL, NULL, NULL, NULL, frc, v, av);
  double e = 0; for (int i = 0; i < n; ++i) e += ae[i];
  printf("%.17g\n", e);
  free(coord); free(at); free(davg); free(dstd); free(ep); free(fp); free(ext); free(et);
  free(mp); free(off); free(cand); free(nl); free(ae); free(frc); free(av);
  return 0;
}
''')
    exe = tmp_path / "drv"
    subprocess.run(["gcc", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-I", src, str(drv), os.path.join(src, "orc_geom.c"), os.path.join(src, "se_e2_a.c"),
                    "-o", str(exe), "-lm"], check=True)
    coord, atype, box = dp.systems.build(0)
    m = dp.model.random_model("water", seed=1000)
    with open(tmp_path / "in.bin", "wb") as f:
        f.write(np.int32(len(atype)).tobytes())
        f.write(coord.tobytes()); f.write(atype.astype(np.int32).tobytes()); f.write(box.tobytes())
        f.write(np.int32(2).tobytes()); f.write(np.array(m["sel"], np.int32).tobytes())
        f.write(np.array([m["rcut"], m["rcut_smth"]]).tobytes())
        f.write(np.array(m["emb"], np.int32).tobytes()); f.write(np.int32(m["axis"]).tobytes())
        f.write(np.array(m["fit"], np.int32).tobytes())
        f.write(np.array([m["davg"].size, m["emb_params"].size, m["fit_params"].size], np.int64).tobytes())
        for k in ("davg", "dstd", "emb_params", "fit_params", "bias_atom_e"):
            f.write(np.ascontiguousarray(m[k], np.float64).tobytes())
    r = subprocess.run([str(exe), str(tmp_path / "in.bin")], capture_output=True, text=True,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=1"})
    assert r.returncode == 0, r.stderr[-2000:]
    assert float(r.stdout) == pytest.approx(367.6157183243399, abs=1e-9)
