"""Compile the gfx950 HIP library ``qste_amd/libqste_hip.so`` with hipcc.

    python -m qste_amd.build          # or __graft_entry__.build()

Each ``csrc/*.hip`` file compiles to an object in ``_build/`` (in parallel),
then one ``hipcc -shared`` link writes the library next to this file, where
``qste_amd.kernels`` loads it.  Flags:

* ``--offload-arch=gfx950``: MI355X only, no other targets.
* ``-ffp-contract=off``: element-wise fp32 arithmetic rounds exactly where
  the specification does (the coordinate step and the encodings are compared
  bit for bit); fused multiply-adds are written out as ``fmaf``.
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE division and sqrt.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-fp32 VALU
  instructions are generated.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc"
BUILD = HERE.parent / "_build"
LIB = HERE / "libqste_hip.so"

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the qste_amd HIP library needs ROCm's hipcc")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{result.stderr[-4000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(SRC.glob("*.hip"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{result.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
