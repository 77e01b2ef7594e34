"""Load the package directory `dpa4c-scale-aware-md_amd` (not an importable
identifier) under the module name `dpamd`, and the CPU oracle."""
import importlib.util
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "dpa4c-scale-aware-md_amd")


def load_pkg():
    if "dpamd" in sys.modules:
        return sys.modules["dpamd"]
    spec = importlib.util.spec_from_file_location(
        "dpamd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["dpamd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import oracle as orc  # noqa: E402
    return orc


def load_dpa4c_oracle():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import dpa4c_oracle  # noqa: E402
    return dpa4c_oracle
