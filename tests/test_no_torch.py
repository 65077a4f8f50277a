"""The product imports without torch (the reference's rule, tests/test_no_torch.py): every module of artlite_amd
imports in a fresh interpreter whose import system refuses torch, and none imports the oracle."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

_SCRIPT = r"""
import importlib, importlib.abc, pkgutil, sys

class Refuse(importlib.abc.MetaPathFinder):
    def find_spec(self, name, path=None, target=None):
        if name.split(".")[0] in ("torch", "oracle"):
            raise ModuleNotFoundError(f"refused: {name}", name=name)
        return None

sys.meta_path.insert(0, Refuse())
import artlite_amd
names = [m.name for m in pkgutil.walk_packages(artlite_amd.__path__, "artlite_amd.")
         if not m.name.rsplit(".", 1)[-1].startswith("lib")]  # (the HIP library is loaded by ctypes)
failed = []
for name in names:
    try:
        importlib.import_module(name)
    except Exception as e:
        failed.append(f"{name}: {type(e).__name__}: {e}")
print(len(names), "modules")
print("\n".join(failed))
sys.exit(1 if failed else 0)
"""


def test_no_torch() -> None:
    r = subprocess.run([sys.executable, "-c", _SCRIPT], capture_output=True, text=True, timeout=300, cwd=ROOT,
                       check=False)
    assert r.returncode == 0, r.stdout + r.stderr
