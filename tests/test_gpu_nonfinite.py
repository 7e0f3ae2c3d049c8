"""NaN and +-Inf through the quantizers and the rotate paths, on the GPU.

The reference reduces each group with torch.amin / torch.amax
(nar/experiment.py:166-167), which propagate NaN: a group holding a NaN gets
scale 1, the canonical NaN zero-point 0x7E00 and code 0; an Inf widens the
range to Inf.  The common path of every kernel reduces with NaN-dropping
fminf/fmaxf and detects NaN elements from their codes; these tests pin the
slow path that then takes over.

* narhip.hooks.dynamic_asym_int4 against the reference's own outputs on the
  27 non-finite golden cases (tests/golden/make_nonfinite_vectors.py): codes,
  scales and zeros bit for bit, dequantized values bit for bit with NaN where
  the reference has NaN.
* ops.rotate_quant on rows holding a NaN, +Inf or -Inf bf16 input through
  every kernel path (block H_128 without and with a per-head rank term, the
  Kronecker transform with the quantizer, the exact rank path, the MFMA rank
  path, the k = 8 full-row fast path): bit-exact against the oracle, which
  propagates NaN and Inf the IEEE way.  On the MFMA rank path an Inf input
  row is left out: the projection u = x V is then +-Inf or NaN in every rank,
  and the three-term bf16 split of an infinite u is (Inf, NaN, NaN), so that
  path returns an all-NaN row where the IEEE correction can keep +-Inf
  entries.  NaN rows are covered on it.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from helpers import f16_bits, to_dev_bf16, to_dev_f32
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from narhip import hooks, ops, workloads  # noqa: E402

NF = np.load(Path(__file__).resolve().parent / "golden" / "nonfinite_vectors.npz")
NF_CASES = [str(k) for k in NF["nf_names"]]

BF16_NAN, BF16_PINF, BF16_NINF = np.uint16(0x7FC0), np.uint16(0x7F80), np.uint16(0xFF80)


@pytest.mark.parametrize("case", NF_CASES)
def test_hooks_quantizer_nonfinite_reference_vectors(case):
    b = int(case.rsplit("_b", 1)[1])
    x = NF[f"{case}_x"]
    deq, s, z, codes = hooks.dynamic_asym_int4(torch.from_numpy(x).cuda(), b)
    torch.cuda.synchronize()
    rows, n = x.shape
    assert np.array_equal(codes.cpu().numpy().reshape(rows, n), NF[f"{case}_codes"].reshape(rows, n))
    assert np.array_equal(f16_bits(s), NF[f"{case}_scale"].reshape(rows, n // b))
    assert np.array_equal(f16_bits(z), NF[f"{case}_zero"].reshape(rows, n // b))
    d = deq.cpu().numpy()
    ref = NF[f"{case}_deq"].reshape(rows, n)
    assert np.array_equal(np.isnan(d), np.isnan(ref)), case
    ok = ~np.isnan(ref)
    assert np.array_equal(d[ok].view(np.uint32), ref[ok].view(np.uint32)), case


def _plant(bits: np.ndarray, value: np.uint16, seed: int) -> np.ndarray:
    """One non-finite element in every other row, at seeded positions."""
    out = bits.copy()
    rng = np.random.default_rng(seed)
    for r in range(0, out.shape[0], 2):
        out[r, rng.integers(out.shape[1])] = value
    return out


PATHS = {
    # name: (workload factory, rank_mode)
    "block128_k0": (lambda: workloads.Workload("b", workloads.e17_8b(tokens=8).x, (1, 128), 32), ops.RANK_AUTO),
    "per_head_k2": (lambda: workloads.kcache_3b(tokens=12), ops.RANK_AUTO),
    "kron_k0": (lambda: workloads.Workload("k", workloads.downproj_8b(tokens=6).x, (28, 512), 128), ops.RANK_AUTO),
    "kron12_k0": (lambda: workloads.Workload("k", workloads.qproj_3b(tokens=6).x, (12, 256), 64), ops.RANK_AUTO),
    "kron_exact_k32": (lambda: workloads.downproj_8b(tokens=6), ops.RANK_EXACT),
    "kron_mfma_k32": (lambda: workloads.downproj_8b(tokens=6), ops.RANK_AUTO),
    "kron_mfma_k16": (lambda: workloads.qproj_3b(tokens=6), ops.RANK_AUTO),
    "block128_k8_fast": (lambda: workloads.e17_8b(tokens=8, k=8), ops.RANK_AUTO),
}


@pytest.mark.parametrize("value", ["nan", "pinf", "ninf"])
@pytest.mark.parametrize("path", list(PATHS))
def test_rotate_quant_nonfinite_rows(path, value):
    factory, mode = PATHS[path]
    if value != "nan" and path.startswith("kron_mfma"):
        pytest.skip("MFMA rank path: an infinite u splits into (Inf, NaN, NaN); NaN rows are covered")
    print(f"[test_rotate_quant_nonfinite_rows] {path} {value}", flush=True)
    w = factory()
    planted = {"nan": BF16_NAN, "pinf": BF16_PINF, "ninf": BF16_NINF}[value]
    bits = _plant(w.x, planted, seed=len(path))
    x = to_dev_bf16(bits)
    codes, scales, zeros = ops.rotate_quant(
        x, hadamard=w.hadamard, v=to_dev_f32(w.v), w_t=to_dev_f32(w.w_t), rank_block=w.rank_block,
        group=w.group, rank_mode=mode)
    torch.cuda.synchronize()
    m, q = w.hadamard
    with np.errstate(invalid="ignore", over="ignore"):
        rot = O.rotate(O.bf16_to_f32(bits), m, q, v=w.v, wt=w.w_t, rank_block=w.rank_block)
        ref = O.quant(rot, w.group)
    c, s, z = codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros)
    planted_rows = np.arange(0, w.tokens, 2)
    other_rows = np.arange(1, w.tokens, 2)
    bad = (c != ref.packed).any(1) | (s != ref.scales).any(1) | (z != ref.zeros).any(1)
    for r in np.nonzero(bad)[0]:
        print(f"   row {r}: codes {(c[r] != ref.packed[r]).sum()} scales {(s[r] != ref.scales[r]).sum()} "
              f"zeros {(z[r] != ref.zeros[r]).sum()}", flush=True)
    # the rows holding a non-finite input: bit for bit on every path
    assert not bad[planted_rows].any(), f"planted rows {np.nonzero(bad)[0].tolist()} differ"
    if path.startswith("kron_mfma"):
        # finite rows of the MFMA rank path: the tie contract of that path
        sub = O.Quantized(*(getattr(ref, f)[other_rows] for f in ("codes", "packed", "scales", "zeros", "deq")))
        rep = O.compare_quant(rot[other_rows], sub, O.unpack(c[other_rows], w.n), s[other_rows], z[other_rows],
                              w.group, rel_err=2.0 ** -21)
        print("  ", rep, flush=True)
        assert rep.code_max_abs_diff <= 1 and rep.code_mismatch_unexplained == 0
        assert rep.scale_mismatch_unexplained == 0 and rep.zero_mismatch_unexplained == 0
    else:
        assert not bad.any(), f"rows {np.nonzero(bad)[0].tolist()} differ"
    # the planted rows really are non-finite after the transform
    assert (~np.isfinite(rot[0])).any()
