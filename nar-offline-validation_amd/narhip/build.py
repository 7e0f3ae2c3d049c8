"""Compile libnarhip.so (HIP kernels + C ABI) for gfx950, in-tree.

The library is a handful of translation units (csrc/abi.hip: the planner and
the extern "C" entry points; csrc/launch_*.hip: the launchers, each of which
instantiates the kernels it launches).  They compile in parallel into
objects under csrc/_build/ and link into narhip/libnarhip.so.

hipcc flags:
  --offload-arch=gfx950          CDNA4 only, no other targets
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                 no packed fp32 VALU forms
  -ffp-contract=off              no implicit a*b+c contraction; fmas are explicit
  -fhip-fp32-correctly-rounded-divide-sqrt, -fno-gpu-flush-denormals-to-zero
                                 IEEE fp32 division and denormals, as the
                                 reference's fp32 arithmetic on the CPU
  -mllvm -amdgpu-mfma-vgpr-form=1
                                 MFMA results in ordinary VGPRs (no accvgpr
                                 moves between the matrix and vector stages)

`build()` always compiles every unit; `build(incremental=True)` recompiles
only units older than a source or header of the csrc directory.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
OBJ = CSRC / "_build"
LIB = PKG / "libnarhip.so"
UNITS = ["abi.hip", "launch_seg.hip", "launch_kron.hip", "launch_rank.hip", "launch_f16.hip", "launch_misc.hip"]
SOURCES = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp"))

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Wno-unused-function",
]


def sources_sha256() -> str:
    """SHA-256 over the kernel and ABI sources (csrc/*.hip, csrc/*.hpp, include/narhip.h, by name): the
    key under which measured profiles (HBM traffic, MFMA utilisation) are filed, so that a profile taken
    on other kernels is recognised as stale."""
    import hashlib
    h = hashlib.sha256()
    for p in SOURCES + [ROOT.parent / "include" / "narhip.h"]:
        h.update(p.name.encode() + b"\0" + p.read_bytes() + b"\0")
    return h.hexdigest()


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def _compile(unit: str, extra: list[str], verbose: bool) -> Path:
    obj = OBJ / (Path(unit).stem + ".o")
    tmp = obj.with_suffix(".o.tmp")
    cmd = [hipcc(), *FLAGS, *extra, "-c", str(CSRC / unit), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(obj)
    return obj


def build(verbose: bool = False, extra: list[str] | None = None, incremental: bool = False,
          jobs: int | None = None) -> Path:
    extra = list(extra or [])
    OBJ.mkdir(exist_ok=True)
    newest_src = max(p.stat().st_mtime for p in SOURCES + [ROOT.parent / "include" / "narhip.h"])
    todo = []
    for unit in UNITS:
        obj = OBJ / (Path(unit).stem + ".o")
        if not incremental or extra or not obj.exists() or obj.stat().st_mtime < newest_src:
            todo.append(unit)
    workers = jobs or min(len(UNITS), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(lambda u: _compile(u, extra, verbose), todo))
    del objs
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[str(OBJ / (Path(u).stem + ".o")) for u in UNITS],
           "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if a not in ("-v", "-i")]
    print(build(verbose="-v" in sys.argv, extra=args, incremental="-i" in sys.argv))
