"""bench.py's host logic: the one-GPU contract and the profile lookups.

The traffic and MFMA figures of the bench line come from rocprofv3 profiles
filed under the SHA-256 of the kernel sources they were measured on; a
profile of other sources must come back as stale (null), and the workload
generators must be the pinned ones (SHA-256 of x, v and w_t of every
workload at a reduced token count, and of the first rows at full size).
"""

from __future__ import annotations

import functools
import hashlib
import importlib.util
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_profile_lookup_by_source_hash(tmp_path):
    b = _bench()
    sha = "ab" * 32
    prof = tmp_path / "t.md"
    prof.write_text("# x\n\n## downproj_8b (8192 x 14336)\n\nKernel sources sha256: " + sha +
                    "\n\n| k | r |\n\nTotal per call: **1234.5 MB**.\n\n## qproj_3b\n\nKernel sources sha256: " +
                    "cd" * 32 + "\n\nTotal per call: **9.0 MB**.\n")
    b.TRAFFIC_SOURCE = prof
    assert b.measured_traffic("downproj_8b", sha) == (1234.5e6, "measured")
    v, status = b.measured_traffic("qproj_3b", sha)
    assert v is None and status.startswith("stale")
    assert b.measured_traffic("kcache_3b", sha)[0] is None
    mu = tmp_path / "m.md"
    mu.write_text("Kernel sources sha256: " + sha + "\n\n| workload | kernel | cycles | MFMA busy | VALU busy |\n"
                  "|---|---|---:|---:|---:|\n| downproj_8b | `proj_mfma_kernel<2>` | 1 | 14.5% | 5.7% |\n"
                  "| downproj_8b | `corr_quant_kernel<128, 1, false, 4>` | 1 | 13.8% | 37.3% |\n")
    b.MFMA_UTIL_SOURCE = mu
    assert b.measured_mfma_busy("downproj_8b", sha) == {"proj_mfma_kernel": 0.145, "corr_quant_kernel": 0.138}
    assert b.measured_mfma_busy("downproj_8b", "00" * 32) is None


# SHA-256 (first 16 hex digits) of x, v, w_t and dest_rows of each generator
# at 64 tokens.  Each generator fills rows in order from its own seeded PCG64
# stream, so these also pin the first 64 rows of the full-size inputs
# (test_prefix_rows_match_full_size checks that on the two smaller shapes).
WORKLOAD_SHA = {
    "kcache_3b": ("66e819951b5aadf2", "cf0afeed4341da9a", "cc150b15c82ff42d", None),
    "qproj_3b": ("7eebf39b61b5eeb2", "d8e5570762fe2bcb", "2d6eea4938a4c76c", None),
    "downproj_8b": ("356a2117d19c0514", "29e43dc4c95d533b", "04b305681a218b1c", None),
    "vcache_decode_8b": ("41c0da719e0fe928", "d1f3c2b2fd75ab55", "95d50f30c5a3fd85", "c2f6b44bec2abc09"),
    "downproj_70b": ("ae98cc2bef856de5", "1514f3f99f04ae5a", "1631dbd3a49a9b01", None),
}


def _sha(a) -> str | None:
    if a is None:
        return None
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


@functools.lru_cache(maxsize=1)
def _digests():
    from narhip import workloads
    out = {}
    for name, make in workloads.CONFIGS.items():
        w = make(64) if name != "vcache_decode_8b" else make(batch=64)
        out[name] = (_sha(w.x), _sha(w.v), _sha(w.w_t), _sha(w.dest_rows))
    return out


@pytest.mark.parametrize("name", ["kcache_3b", "qproj_3b", "downproj_8b", "vcache_decode_8b", "downproj_70b"])
def test_workload_generators_pinned(name):
    got = _digests()[name]
    want = WORKLOAD_SHA.get(name)
    assert want is not None, f"no pin for {name}: {got}"
    assert got == want, f"{name}: generator output changed: {got} != {want}"


def test_prefix_rows_match_full_size():
    from narhip import workloads
    for name in ("kcache_3b", "qproj_3b"):
        small, full = workloads.CONFIGS[name](64), workloads.CONFIGS[name]()
        assert np.array_equal(small.x, full.x[:64]), name
