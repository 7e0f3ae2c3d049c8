"""Compile libnarhip.so (HIP kernels + C ABI) for gfx950, in-tree.

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
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
LIB = PKG / "libnarhip.so"
SOURCES = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp"))

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, *(extra or []), str(CSRC / "abi.hip"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, extra=[a for a in sys.argv[1:] if a != "-v"]))
