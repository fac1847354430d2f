"""Test configuration: loads the package, registers the `gpu` marker.

The package directory is `prefree-public_amd/` (not an importable name), so it
is loaded by path and registered as `prefree_amd`.  Native libraries are built
only when they are missing (build with __graft_entry__.build() after a change).

PF_AUTO's tests check its built-in rules: the tuning table that ships with the
library (loaded by default) is switched off here with an empty
$PREFREE_TUNING_TABLE; the tests of the table load it explicitly.
"""
import importlib.util
import os
import subprocess
import sys

os.environ["PREFREE_TUNING_TABLE"] = ""

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "prefree-public_amd")
if REPO not in sys.path:
    sys.path.insert(0, REPO)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def _ensure_built():
    need = [os.path.join(PKG_DIR, "lib", "libprefree.so"), os.path.join(REPO, "oracle", "liboracle.so")]
    if all(os.path.exists(p) for p in need):
        return
    subprocess.run(["make", "-C", os.path.join(REPO, "oracle")], check=True)
    subprocess.run(["make", "-C", PKG_DIR, "-j4"], check=True)


def _load_pkg():
    if "prefree_amd" in sys.modules:
        return sys.modules["prefree_amd"]
    spec = importlib.util.spec_from_file_location("prefree_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["prefree_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


_ensure_built()
_load_pkg()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; run with -m gpu on a machine that has one")
