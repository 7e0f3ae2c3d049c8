"""Whole-tensor parity of the default (auto) path on the five full workloads.

The parity bound is a statistic over the whole tensor: codes equal, or +-1
only at rounding ties, scales and zeros equal or one fp16 ulp apart only at
ties, such tie mismatches on at most 0.01% of the codes / groups (the E17
Verification-B protocol, nar/e17_v2.py:79-116,204-210, tightened to ties).

The reference for every row is the exact path (rank_mode=EXACT: every BLAS
product of the reference as an fp64 sum rounded once, as the oracle defines
it), whose fp32 rotated rows, codes, scales and zeros are first re-confirmed
bit for bit against the oracle on 1024 rows (the first 512 and 512 seeded
ones).  Then the auto path's codes, scales and zeros are classified against
the exact path's over all rows with the oracle's comparator, in chunks of
rows, and the mismatch counts are printed.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits, to_dev_bf16, to_dev_f32
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from narhip import ops, workloads  # noqa: E402

REL_ERR = 2.0 ** -21      # bound of the MFMA path's rotated rows (|x'| + row rms)
CHUNK = 512


def _run(w, x, v, wt, dest, mode, rotated=None):
    codes, scales, zeros = ops.rotate_quant(
        x, hadamard=w.hadamard, v=v, w_t=wt, rank_block=w.rank_block, group=w.group, rotated=rotated,
        dest_rows=dest, rank_mode=mode, out_rows=w.out_rows)
    torch.cuda.synchronize()
    if dest is not None:
        codes, scales, zeros = codes[dest], scales[dest], zeros[dest]
    return codes, scales, zeros


@pytest.mark.parametrize("name", list(workloads.CONFIGS))
def test_whole_tensor_auto_against_exact(name):
    print(f"[test_whole_tensor_auto_against_exact] {name}: generating", flush=True)
    w = workloads.CONFIGS[name]()
    T, n, b = w.tokens, w.n, w.group
    x = to_dev_bf16(w.x)
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    dest = None if w.dest_rows is None else torch.from_numpy(w.dest_rows).cuda()
    rot = torch.empty((T, n), dtype=torch.float32, device="cuda")
    ce, se, ze = _run(w, x, v, wt, dest, ops.RANK_EXACT, rotated=rot)
    ca, sa, za = _run(w, x, v, wt, dest, ops.RANK_AUTO)
    print(f"   {name}: {T} x {n}, k={w.k}, b={b}; kernels done", flush=True)

    # 1. the exact path against the oracle on 1024 rows
    rng = np.random.default_rng(11)
    if T > 1024:
        rows = np.concatenate([np.arange(512), 512 + np.sort(rng.choice(T - 512, size=512, replace=False))])
    else:
        rows = np.arange(T)
    m, q = w.hadamard
    for i in range(0, rows.size, 256):
        sel = rows[i:i + 256]
        ref_rot = O.rotate(O.bf16_to_f32(w.x[sel]), m, q, v=w.v, wt=w.w_t, rank_block=w.rank_block)
        ref = O.quant(ref_rot, b)
        idx = torch.from_numpy(sel).cuda()
        assert np.array_equal(rot[idx].cpu().numpy(), ref_rot), f"exact rotated rows differ near row {sel[0]}"
        assert np.array_equal(ce[idx].cpu().numpy(), ref.packed)
        assert np.array_equal(f16_bits(se[idx]), ref.scales) and np.array_equal(f16_bits(ze[idx]), ref.zeros)
    print(f"   {name}: exact path == oracle on {rows.size} rows", flush=True)

    # 2. the auto path against the exact path, every row
    totals = dict(elements=0, groups=0, code_mismatch=0, code_mismatch_unexplained=0, code_max_abs_diff=0,
                  scale_mismatch=0, scale_mismatch_unexplained=0, zero_mismatch=0, zero_mismatch_unexplained=0)
    for r0 in range(0, T, CHUNK):
        r1 = min(T, r0 + CHUNK)
        xr = rot[r0:r1].cpu().numpy()
        codes_e = ce[r0:r1].cpu().numpy()
        ref = O.Quantized(O.unpack(codes_e, n), codes_e, f16_bits(se[r0:r1]), f16_bits(ze[r0:r1]), None)
        rep = O.compare_quant(xr, ref, O.unpack(ca[r0:r1].cpu().numpy(), n), f16_bits(sa[r0:r1]),
                              f16_bits(za[r0:r1]), b, rel_err=REL_ERR)
        for key in totals:
            val = getattr(rep, key)
            totals[key] = max(totals[key], val) if key == "code_max_abs_diff" else totals[key] + val
        if (r0 // CHUNK) % 8 == 0:
            print(f"   {name}: rows {r0}..{r1 - 1} classified", flush=True)
    total = O.ParityReport(**totals)
    print(f"   {name} whole tensor: {total}; code mismatch fraction {total.code_mismatch_fraction:.2e}, "
          f"scale/zero mismatch fraction {total.meta_mismatch_fraction:.2e}", flush=True)
    assert total.within_contract(), total
