"""Wheel packaging (setup.py): the metadata is readable without a build, and the
library the ctypes loader looks for is the one the package data ships."""

from __future__ import annotations

import ast
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_setup_metadata_without_building():
    out = subprocess.run([sys.executable, "setup.py", "--name", "--version"], cwd=ROOT, check=True,
                         capture_output=True, text=True).stdout.split()
    import skmetal_amd._about as about

    assert out == ["skmetal-amd", about.__version__]


def test_package_data_ships_the_loaded_library():
    tree = ast.parse((ROOT / "setup.py").read_text())
    call = next(n for n in ast.walk(tree) if isinstance(n, ast.Call) and getattr(n.func, "id", "") == "setup")
    kw = {k.arg: k.value for k in call.keywords}
    data = ast.literal_eval(kw["package_data"])
    from skmetal_amd import _bridge

    assert _bridge.LIB_NAME in data["skmetal_amd"]
    assert set(ast.literal_eval(kw["packages"])) == {"skmetal_amd", "skmetal_amd.estimators"}
