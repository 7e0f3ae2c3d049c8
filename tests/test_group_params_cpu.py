"""The two divisions of the quantizer's group parameters, as the kernels compute them.

raw = (hi - lo) / 15 must be the correctly rounded fp32 quotient of the
reference (nar/experiment.py:169): the kernels use Markstein's correction
step q1 = fma(fma(-q0, 15, d), RN(1/15), q0) from q0 = d * RN(1/15).
rs = RN(1/s) feeds the reciprocal quantizer path: one Newton step from the
hardware reciprocal.  tests/native/group_params_check.c performs the same
fp32 operations (fmaf, -ffp-contract=off) over every non-negative fp32 range
d and every fp16 scale s (with the reciprocal one ulp off either way), and the
planted mistake (no correction step) must fail both scans.
"""

from __future__ import annotations

import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent


def _scan(naive: bool = False, stride: int = 8) -> dict[str, tuple[int, int]]:
    with tempfile.TemporaryDirectory() as tmp:
        exe = Path(tmp) / "group_params_check"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                        str(HERE / "native" / "group_params_check.c"), "-lm"], check=True)

        def run(phase: int) -> str:
            args = [str(exe), str(stride), str(phase)] + (["naive"] if naive else [])
            return subprocess.run(args, check=True, capture_output=True, text=True).stdout

        with ThreadPoolExecutor(max_workers=8) as pool:
            outs = list(pool.map(run, range(stride)))
    tot: dict[str, list[int]] = {}
    for out in outs:
        for line in out.splitlines():
            name, bad, checked = line.split()
            acc = tot.setdefault(name, [0, 0])
            acc[0] += int(bad)
            acc[1] += int(checked)
    return {k: (v[0], v[1]) for k, v in tot.items()}


def test_div15_and_reciprocal_exhaustive():
    res = _scan()
    assert res["div15"] == (0, 2 ** 31)
    # the reciprocal scan runs once per phase over all fp16 scales
    assert res["recip"][0] == 0 and res["recip"][1] == 8 * 3 * 31743


def test_dropping_the_correction_steps_fails():
    res = _scan(naive=True, stride=64)
    assert res["div15"][0] > 0
    assert res["recip"][0] > 0
