"""CPU checks that the product path stands on the HIP library alone: no
module of the package imports the CPU oracle (test infrastructure), importing
every module of it loads none, and a missing library is an error rather than
a fallback."""

import pathlib
import re
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG = ROOT / "vla-to-npu_amd" / "smolvla"


def test_no_package_module_names_the_oracle():
    pat = re.compile(r"^\s*(from|import)\s+oracle\b|smolvla_ref", re.M)
    hits = [str(f.relative_to(ROOT)) for f in PKG.rglob("*.py") if pat.search(f.read_text())]
    assert hits == []


def test_importing_every_package_module_loads_no_oracle_module():
    code = (
        "import importlib, pkgutil, sys\n"
        f"sys.path.insert(0, {str(ROOT / 'vla-to-npu_amd')!r})\n"
        "import smolvla\n"
        "for m in pkgutil.walk_packages(smolvla.__path__, 'smolvla.'):\n"
        "    if m.name not in ('smolvla.build', 'smolvla.libsvla'):\n"
        "        importlib.import_module(m.name)\n"
        "bad = [n for n in sys.modules if n == 'oracle' or n.startswith('oracle.')]\n"
        "print(len([n for n in sys.modules if n.startswith('smolvla')]), bad)\n"
        "sys.exit(1 if bad else 0)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                       cwd=str(ROOT / "tests"))
    assert r.returncode == 0, r.stdout + r.stderr


def test_missing_library_is_an_error(tmp_path):
    from smolvla import _lib
    saved = _lib._LIB
    _lib._LIB = None
    try:
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            _lib.load(tmp_path / "libsvla.so")
    finally:
        _lib._LIB = saved
