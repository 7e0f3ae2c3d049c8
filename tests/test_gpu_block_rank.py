"""GPU parity of the block-H_128, full-row k <= 8, group-128 rotate-quant path
(proj_tok + xform128 with the INT4 epilogue: E17's k = 8 setting).

Called without a rotated output (which selects these kernels), against the
oracle's rotate + quantizer with the tie-aware contract of the MFMA tests at a
1-ulp rotated bound (the fp64 projection sums differ from the oracle's only in
order); expected exact.  Covers ranks 1..8, ragged token counts, a width that
is not a multiple of 2048 channels, Hadamard input signs, destination-row
scatter and caller partials (Kernel B after launch_projection_dot).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import ops, workloads  # noqa: E402

REL_ERR = 2.0 ** -22


def factors(n, k, seed):
    rng = np.random.default_rng(seed)
    v = np.ascontiguousarray(workloads.orthonormal(rng, n, k))
    wt = np.ascontiguousarray(-workloads.orthonormal(rng, n, k).T)
    return v, wt


def rows(t, n, seed):
    x = workloads._silu_up(seed, t, n, 16)
    return workloads.bf16_bits(x)


def check(xbits, codes, scales, zeros, v, wt, signs=None, label=""):
    n = xbits.shape[1]
    rot = O.rotate(O.bf16_to_f32(xbits), 1, 128, signs=signs, v=v, wt=wt)
    ref = O.quant(rot, 128)
    rep = O.compare_quant(rot, ref, O.unpack(codes, n), scales, zeros, 128, rel_err=REL_ERR)
    print(f"  {label}: {rep}", flush=True)
    assert rep.within_contract(), rep
    return rep


def dev_bf16(bits):
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)


@pytest.mark.parametrize("t,n,k", [(77, 8192, 8), (64, 14336, 1), (130, 3072, 3), (1, 8192, 5)])
def test_ranks_and_shapes(t, n, k):
    print(f"[test_ranks_and_shapes] t={t} n={n} k={k}", flush=True)
    xb = rows(t, n, 40 + k)
    v, wt = factors(n, k, k)
    codes, scales, zeros = ops.rotate_quant(dev_bf16(xb), hadamard=(1, 128), v=torch.from_numpy(v).cuda(),
                                            w_t=torch.from_numpy(wt).cuda(), group=128)
    torch.cuda.synchronize()
    rep = check(xb, codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros), v, wt, label=f"k={k}")
    assert rep.code_mismatch == 0 and rep.scale_mismatch == 0 and rep.zero_mismatch == 0


def test_signs_and_destination_rows():
    print("[test_signs_and_destination_rows]", flush=True)
    t, n, k = 48, 8192, 8
    xb = rows(t, n, 7)
    v, wt = factors(n, k, 7)
    signs = np.random.default_rng(7).choice(np.array([-1.0, 1.0], np.float32), size=n)
    dest = np.random.default_rng(8).choice(200, size=t, replace=False).astype(np.int64)
    codes = torch.zeros((200, n // 2), dtype=torch.uint8, device="cuda")
    scales = torch.zeros((200, n // 128), dtype=torch.float16, device="cuda")
    zeros = torch.zeros((200, n // 128), dtype=torch.float16, device="cuda")
    ops.rotate_quant(dev_bf16(xb), hadamard=(1, 128), signs=torch.from_numpy(signs).cuda(),
                     v=torch.from_numpy(v).cuda(), w_t=torch.from_numpy(wt).cuda(), group=128, codes=codes,
                     scales=scales, zeros=zeros, dest_rows=torch.from_numpy(dest).cuda())
    torch.cuda.synchronize()
    c, s, z = codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros)
    rep = check(xb, c[dest], s[dest], z[dest], v, wt, signs=signs, label="signs + dest")
    assert rep.code_mismatch == 0
    untouched = np.setdiff1d(np.arange(200), dest)
    assert not c[untouched].any() and not s[untouched].any()


@pytest.mark.parametrize("splits", [1, 4])
def test_caller_partials(splits):
    """Kernel A then Kernel B: partials [T, splits*k] folded in split order."""
    print(f"[test_caller_partials] splits={splits}", flush=True)
    t, n, k = 96, 14336, 8
    xb = rows(t, n, 9)
    v, wt = factors(n, k, 9)
    x = dev_bf16(xb)
    vd, wd = torch.from_numpy(v).cuda(), torch.from_numpy(wt).cuda()
    partial = torch.empty((t, splits * k), dtype=torch.float32, device="cuda")
    ops.rank_projection(x, vd, partial, ops.RANK_EXACT)
    codes = torch.empty((t, n // 2), dtype=torch.uint8, device="cuda")
    scales = torch.empty((t, n // 128), dtype=torch.float16, device="cuda")
    zeros = torch.empty_like(scales)
    ops.group_quant(x, partial, wd, codes, scales, zeros, hadamard=(1, 128), group=128)
    torch.cuda.synchronize()
    check(xb, codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros), v, wt, label=f"partials S={splits}")
