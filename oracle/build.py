"""Build the CPU oracle (test infrastructure) into oracle/_build/.

gcc -O2 with contraction and fast-math disabled, so every fp32 operation in
nar_oracle.c is one IEEE round-to-nearest-even operation as written.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "nar_oracle.c"
OUT = HERE / "_build" / "libnar_oracle.so"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
           "-fno-fast-math", "-frounding-math", "-Wall", "-Wextra",
           str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
