"""The two division shortcuts of the device kernels, checked on the CPU.

* FWHT normalisation: RN(v / fp32(sqrt(Q))) through a reciprocal and two fma
  corrections, with the IEEE division for |v| < 2^-100
  (csrc/narhip_device.hpp, div_sqrt_q); for Q = 128 and 512 as
  fma(v, HI, v * LO) with 1/c split in two fp32 pieces, with the division for
  |v| < 2^-90.  tests/native/div_sqrt_check.c runs the same fp32 operations;
  this test scans every finite fp32 pattern for the widths the kernels divide
  by (128 and 512 split, 2048 and 8192), in 8 processes, and a strided subset
  for the other widths (NARHIP_FULL_DIV_SCAN=1 scans all of them).
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
QS = (2, 8, 12, 28, 32, 128, 512, 2048, 8192)


# widths the kernels divide by with the reciprocal-and-correction form: every
# finite fp32 pattern is scanned (8 processes); the other widths on a stride
KERNEL_QS = (2048, 8192)


def _parallel_scan(exe: Path, args_of_phase) -> list[list[int]]:
    procs = [subprocess.Popen([str(exe), *args_of_phase(ph)], stdout=subprocess.PIPE, text=True)
             for ph in range(8)]
    outs = [p.communicate()[0] for p in procs]
    assert all(p.returncode == 0 for p in procs)
    return [list(map(int, o.split())) for o in outs]


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
        if not full:
            for q in KERNEL_QS:
                parts = _parallel_scan(exe, lambda ph: ["8", str(ph), str(q)])
                bad = sum(p[1] for p in parts)
                checked = sum(p[2] for p in parts)
                assert checked > 4_000_000_000, q
                assert bad == 0, f"Q={q}: {bad} mismatches over every finite pattern"


def _split_constants():
    """(Q, HI, LO) of RecipSqrtQ in the device header, as C float literals."""
    text = (HERE.parent / "nar-offline-validation_amd" / "csrc" / "narhip_device.hpp").read_text()
    import re
    found = re.findall(r"struct RecipSqrtQ<(\d+)> \{[^}]*?hi = ([0-9a-fx.p+-]+)f, lo = ([0-9a-fx.p+-]+)f;", text)
    return [(int(q), hi, lo) for q, hi, lo in found]


def test_split_constants_are_the_reciprocal_split():
    consts = _split_constants()
    assert sorted(q for q, _, _ in consts) == [128, 512]
    for q, hi, lo in consts:
        c = np.float32(np.sqrt(np.float64(q)))
        r = 1.0 / np.float64(c)
        want_hi = np.float32(r)
        want_lo = np.float32(r - np.float64(want_hi))
        assert np.float32(float.fromhex(hi)) == want_hi, q
        assert np.float32(float.fromhex(lo)) == want_lo, q


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_split_division_matches_ieee_division():
    full = os.environ.get("NARHIP_FULL_DIV_SCAN") == "1"
    with tempfile.TemporaryDirectory() as tmp:
        exe = Path(tmp) / "div_sqrt_check"
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-frounding-math", "-o", str(exe),
                        str(HERE / "native" / "div_sqrt_check.c"), "-lm"], check=True)
        def scan(q, hi, lo, stride=4099, phase=17):
            out = subprocess.run([str(exe), "split", str(stride), str(phase), str(q), hi, lo],
                                 check=True, capture_output=True, text=True).stdout.split()
            return int(out[1]), int(out[2])

        def scan_all(q, hi, lo):
            parts = _parallel_scan(exe, lambda ph: ["split", "8", str(ph), str(q), hi, lo])
            return sum(p[1] for p in parts), sum(p[2] for p in parts)

        for q, hi, lo in _split_constants():
            bad, checked = (scan(q, hi, lo, 1, 0) if full else scan_all(q, hi, lo))
            assert checked > 1_000_000
            assert bad == 0, f"Q={q}: {bad} mismatches"
            # a dropped low piece (plain multiplication by RN(1/c)) is caught
            bad0, _ = scan(q, hi, "0")
            assert bad0 > 0, q


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
