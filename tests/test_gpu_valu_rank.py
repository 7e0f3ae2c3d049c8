"""GPU parity of the full-row rank path on fp64 VALU (k < 16, rank_mode auto).

The projection runs over channel splits with fp64 partial sums folded once,
and the correction sums the k products of each channel in fp64; both round
once to fp32 like the oracle, differing from it only in the order of the fp64
additions.  Checked with the tie-aware contract of the MFMA paths (it is
expected to be met with zero mismatches), on the reference's E17 block-H_128
setting and on a Kronecker row.
"""

from __future__ import annotations

import numpy as np
import pytest

from test_gpu_mfma import check_contract, run_mfma

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import ops, workloads  # noqa: E402


@pytest.mark.parametrize("tokens,k", [(40, 8), (37, 4), (33, 12)])
def test_block_h128_full_row_small_rank(tokens, k):
    print(f"[test_block_h128_full_row_small_rank] tokens={tokens} k={k}", flush=True)
    w = workloads.e17_3b(tokens=tokens, k=8)
    if k != 8:
        w.v = np.ascontiguousarray(workloads.orthonormal(np.random.default_rng(k), w.n, k))
        w.w_t = np.ascontiguousarray(-workloads.orthonormal(np.random.default_rng(100 + k), w.n, k).T)
    codes, scales, zeros, rot = run_mfma(w, rank_mode=ops.RANK_AUTO)
    rep = check_contract(w, codes, scales, zeros, rot, label=f"e17_3b T={tokens} k={k}")
    assert rep.code_mismatch == 0 and rep.scale_mismatch == 0 and rep.zero_mismatch == 0


def test_e17_8b_k8_sampled_rows():
    print("[test_e17_8b_k8_sampled_rows]", flush=True)
    w = workloads.e17_8b(tokens=256, k=8)
    codes, scales, zeros, rot = run_mfma(w, rank_mode=ops.RANK_AUTO)
    rows = np.array([0, 1, 63, 128, 200, 255])
    check_contract(w, codes, scales, zeros, rot, rows=rows, label="e17_8b k=8")


def test_kronecker_row_small_rank():
    print("[test_kronecker_row_small_rank]", flush=True)
    w = workloads.downproj_8b(tokens=12)
    w.v = np.ascontiguousarray(w.v[:, :8])
    w.w_t = np.ascontiguousarray(w.w_t[:8])
    codes, scales, zeros, rot = run_mfma(w, rank_mode=ops.RANK_AUTO)
    check_contract(w, codes, scales, zeros, rot, label="H28xH512 k=8")
