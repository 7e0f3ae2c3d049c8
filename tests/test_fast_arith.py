"""The two division shortcuts of the device kernels, checked on the CPU.

* FWHT normalisation: RN(v / fp32(sqrt(Q))) through a reciprocal and two fma
  corrections, with the IEEE division for |v| < 2^-100
  (csrc/narhip_device.hpp, div_sqrt_q).  tests/native/div_sqrt_check.c runs
  the same fp32 operations; this test scans a strided subset of all 2^32 bit
  patterns (NARHIP_FULL_DIV_SCAN=1 scans all of them).
* Quantizer: rint((x - z) * RN(1/s)) with the exact division only for lanes
  within 2^-18 of a half-integer (quant_code_fast).  Checked against
  rint(RN((x - z) / s)) on random groups and on constructed near-ties.
"""

import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
QS = (2, 8, 12, 28, 32, 128, 512, 2048)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_div_sqrt_matches_ieee_division():
    full = os.environ.get("NARHIP_FULL_DIV_SCAN") == "1"
    with tempfile.TemporaryDirectory() as tmp:
        exe = Path(tmp) / "div_sqrt_check"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-frounding-math", "-o", str(exe),
                        str(HERE / "native" / "div_sqrt_check.c"), "-lm"], check=True)
        stride, phase = (1, 0) if full else (4099, 17)
        out = subprocess.run([str(exe), str(stride), str(phase), *map(str, QS)], check=True,
                             capture_output=True, text=True).stdout
    rows = [tuple(map(int, line.split())) for line in out.strip().splitlines()]
    assert [r[0] for r in rows] == list(QS)
    for q, bad, checked in rows:
        assert checked > 1_000_000
        assert bad == 0, f"Q={q}: {bad} mismatches"


def _exact_codes(x, z, s):
    d = (x - z).astype(np.float32)
    return np.clip(np.rint((d / s).astype(np.float32)), 0, 15)


def _fast_codes(x, z, s):
    rs = (np.float32(1.0) / s).astype(np.float32)
    y = ((x - z).astype(np.float32) * rs).astype(np.float32)
    r = np.rint(y)
    tie = np.abs(y - r) >= np.float32(0.5 - 2.0 ** -18)
    return np.clip(r, 0, 15), tie


def _fp16_round(a):
    return a.astype(np.float16).astype(np.float32)


def test_fast_quantizer_equals_division():
    rng = np.random.default_rng(20260902)
    mismatches = 0
    flagged = 0
    total = 0
    for scale in (1e-3, 1.0, 37.0, 1e4):
        x = (rng.standard_normal((4096, 128)) * scale).astype(np.float32)
        lo, hi = x.min(axis=1, keepdims=True), x.max(axis=1, keepdims=True)
        s = _fp16_round(((hi - lo) / np.float32(15)).astype(np.float32))
        z = _fp16_round(lo)
        exact = _exact_codes(x, z, s)
        fast, tie = _fast_codes(x, z, s)
        mismatches += int(np.count_nonzero((exact != fast) & ~tie))
        flagged += int(np.count_nonzero(tie))
        total += x.size
    assert mismatches == 0
    assert flagged < total * 1e-4


def test_fast_quantizer_flags_constructed_ties():
    # x = z + (k + 1/2) * s exactly, and its fp32 neighbours: every one must be
    # flagged or rounded like the division.
    rng = np.random.default_rng(7)
    s = _fp16_round(rng.uniform(1e-3, 10.0, 20000).astype(np.float32))
    z = _fp16_round(rng.uniform(-50.0, 50.0, 20000).astype(np.float32))
    k = rng.integers(0, 15, 20000).astype(np.float32)
    x0 = (z.astype(np.float64) + (k + 0.5) * s.astype(np.float64)).astype(np.float32)
    for ulps in range(-3, 4):
        x = x0.copy()
        step = np.inf if ulps > 0 else -np.inf
        for _ in range(abs(ulps)):
            x = np.nextafter(x, np.float32(step))
        exact = _exact_codes(x, z, s)
        fast, tie = _fast_codes(x, z, s)
        assert not np.any((exact != fast) & ~tie), f"unflagged mismatch at {ulps} ulp"
