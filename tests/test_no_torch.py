"""The product stays free of torch and of the test oracle (the reference's no-torch rule for its package,
tests/test_no_torch.py there; here also: the oracle is test infrastructure only).

Two independent checks: a static one (every ``import`` statement of every source file under ``artlite_amd/``, parsed
with ``ast``) and a dynamic one (a fresh interpreter in which ``torch`` and ``oracle`` are poisoned entries of
``sys.modules``, so that importing them raises, imports each module file of the package and then finds neither
among the loaded modules)."""

import ast
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "artlite_amd"
BANNED = ("torch", "oracle")


def _modules() -> list[str]:
    """Dotted names of the package's Python modules (the HIP library is loaded by ctypes, not imported)."""
    out = []
    for f in sorted(PKG.rglob("*.py")):
        rel = f.relative_to(ROOT).with_suffix("")
        parts = list(rel.parts)
        if parts[-1] == "__init__":
            parts.pop()
        out.append(".".join(parts))
    return out


def test_no_banned_import_statements() -> None:
    """No source file of the package names torch or the oracle in an import statement (also inside functions)."""
    offenders = []
    for f in sorted(PKG.rglob("*.py")):
        for node in ast.walk(ast.parse(f.read_text(), str(f))):
            if isinstance(node, ast.Import):
                names = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom) and node.level == 0 and node.module:
                names = [node.module]
            else:
                continue
            offenders += [f"{f.relative_to(ROOT)}:{node.lineno}: {n}" for n in names if n.split(".")[0] in BANNED]
    assert not offenders, offenders


_PROBE = """
import importlib, sys
for name in {banned!r}:
    sys.modules[name] = None  # (import of a None entry raises ImportError)
bad = []
for mod in {mods!r}:
    try:
        importlib.import_module(mod)
    except Exception as e:
        bad.append(mod + ": " + type(e).__name__ + ": " + str(e))
loaded = sorted(m for m, v in sys.modules.items() if v is not None and m.split(".")[0] in {banned!r})
print("imported", len({mods!r}), "modules; loaded banned:", loaded)
print(*bad, sep=chr(10))
sys.exit(1 if bad or loaded else 0)
"""


def test_package_imports_without_torch() -> None:
    mods = _modules()
    assert "artlite_amd.moe.layer" in mods and "artlite_amd.gguf_model" in mods
    r = subprocess.run([sys.executable, "-c", _PROBE.format(banned=BANNED, mods=mods)], capture_output=True, text=True,
                       timeout=300, cwd=ROOT, check=False)
    assert r.returncode == 0, r.stdout + r.stderr
