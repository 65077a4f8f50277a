"""Build ``artlite_amd/libartlite_moe.so`` from ``artlite_amd/csrc/*.hip`` with hipcc for gfx950.

``python -m artlite_amd.build`` (or ``build()``) compiles every source each time it is called (objects under
``artlite_amd/csrc/_build``), then links the shared library in place, next to this file. No torch involved."""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libartlite_moe.so"
ARCH = "gfx950"

# all device code: gfx950 only; packed fp32 instructions off (they are not trusted on the target pool)
COMMON = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-Wall", "-Wno-unused-result"]
# per-file extra flags: the dequantizer's fp32 operations in the reference's order, unfused; the prefill tiles with the
# machine scheduler's ILP strategy (it issues a stage's LDS reads ahead of the MFMAs that use them, where the default
# strategy, chasing an occupancy these one-wave-per-SIMD kernels cannot have, reads each operand right before its use)
EXTRA = {"dequant.hip": ["-ffp-contract=off"], "route.hip": ["-ffp-contract=off"],
         "prefill.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]}


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build artlite_amd)")


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    noise = [ln for ln in r.stderr.splitlines() if ln.strip() and "not a recognized feature" not in ln]
    if noise:
        print("\n".join(noise), file=sys.stderr)


def build(verbose: bool = False, jobs: int = 8) -> Path:
    cc = hipcc()
    obj_dir = CSRC / "_build"
    obj_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [obj_dir / (s.stem + ".o") for s in sources]

    def compile_one(i: int) -> None:
        cmd = [cc, *COMMON, *EXTRA.get(sources[i].name, []), "-c", str(sources[i]), "-o", str(objs[i])]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)

    with ThreadPoolExecutor(max(1, min(jobs, len(sources)))) as ex:
        list(ex.map(compile_one, range(len(sources))))
    tmp = OUT.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
