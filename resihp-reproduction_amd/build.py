"""Build the gfx950 HIP library ``libresihp_hip.so`` in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``_build/`` (in parallel),
then linked into ``resihp/libresihp_hip.so`` next to the Python package that
loads it.  ``python build.py`` or ``build()`` from Python; no cmake.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "resihp" / "libresihp_hip.so"
ARCH = os.environ.get("RESIHP_HIP_ARCH", "gfx950")

# -packed-fp32-ops: hipcc must not emit packed fp32 math on this target.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _compile(src: Path, hipcc: str) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library; return its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2)), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, hipcc), sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
