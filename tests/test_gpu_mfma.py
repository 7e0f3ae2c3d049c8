"""GPU parity of the MFMA paths (Paley product and rank-k on bf16 MFMA).

The MFMA stages compute the reference's BLAS products in a different order
than the oracle's fp64 definition, so the contract is the tie-aware one:
  * rotated fp32 rows within REL_ERR of the oracle, relative to |x'| + row rms
  * INT4 codes equal, or +-1 only where the oracle's quotient lies within that
    error of a rounding tie; scales/zeros equal or 1 fp16 ulp apart only where
    the oracle's pre-rounding value lies within that error of an fp16 midpoint;
    such tie mismatches on at most 0.01% of codes / groups.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits, oracle_for, to_dev_bf16, to_dev_f32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import ops, workloads  # noqa: E402

REL_ERR = 2.0 ** -21      # bound on |x'_mfma - x'_oracle| / (|x'| + row rms)


def test_mfma_operand_mapping():
    """D[4g+i][l%16] = sum over slots of A(row l%16) * B(col l%16), g = l/16."""
    print("[test_mfma_operand_mapping]", flush=True)
    rng = np.random.default_rng(1)
    a = rng.integers(-4, 5, size=(64, 8)).astype(np.float32)
    b = rng.integers(-4, 5, size=(64, 8)).astype(np.float32)
    d = ops.mfma_probe(torch.from_numpy(a).cuda().bfloat16(), torch.from_numpy(b).cuda().bfloat16())
    torch.cuda.synchronize()
    d = d.cpu().numpy()
    A = np.zeros((16, 32)); B = np.zeros((32, 16))
    for lane in range(64):
        g, c = lane // 16, lane % 16
        A[c, 8 * g:8 * g + 8] = a[lane]
        B[8 * g:8 * g + 8, c] = b[lane]
    D = A @ B
    want = np.array([[D[4 * (lane // 16) + i, lane % 16] for i in range(4)] for lane in range(64)])
    assert np.array_equal(d, want)


def run_mfma(w, prepared=None, rank_mode=ops.RANK_AUTO, x=None):
    x = to_dev_bf16(w.x) if x is None else x
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    rot = torch.empty((w.tokens, w.n), dtype=torch.float32, device="cuda")
    codes, scales, zeros = ops.rotate_quant(x, hadamard=w.hadamard, v=v, w_t=wt, prepared=prepared,
                                            rank_block=w.rank_block, group=w.group, rotated=rot,
                                            rank_mode=rank_mode)
    torch.cuda.synchronize()
    return codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros), rot.cpu().numpy()


def check_contract(w, codes, scales, zeros, rot, rows=None, label=""):
    ref_rot, ref = oracle_for(w, rows)
    if rows is not None:
        codes, scales, zeros, rot = codes[rows], scales[rows], zeros[rows], rot[rows]
    err = O.rotated_error(rot, ref_rot)
    rep = O.compare_quant(ref_rot, ref, O.unpack(codes, w.n), scales, zeros, w.group, rel_err=REL_ERR)
    print(f"  {label}: rotated err {err:.3e} ({err / 2**-24:.2f} ulp-units), {rep}", flush=True)
    assert err <= REL_ERR, err
    assert rep.within_contract(), rep
    deq = O.dequant(codes, scales, zeros, w.n, w.group)
    nm_obs, nm_ref = O.nmse(ref_rot, deq), O.nmse(ref_rot, ref.deq)
    assert f"{nm_obs:.4g}" == f"{nm_ref:.4g}", (nm_obs, nm_ref)
    return rep


SMALL = {
    "qproj_3b": lambda: workloads.qproj_3b(tokens=200),
    "downproj_8b": lambda: workloads.downproj_8b(tokens=96),
    "downproj_70b": lambda: workloads.downproj_70b(tokens=24),
}


@pytest.mark.parametrize("name", list(SMALL))
def test_small_mfma_contract(name):
    print(f"[test_small_mfma_contract] {name}", flush=True)
    w = SMALL[name]()
    check_contract(w, *run_mfma(w), label=name)


@pytest.mark.parametrize("name", ["qproj_3b", "downproj_8b", "downproj_70b"])
def test_full_size_mfma_sampled(name):
    print(f"[test_full_size_mfma_sampled] {name}", flush=True)
    w = workloads.CONFIGS[name]()
    codes, scales, zeros, rot = run_mfma(w)
    # seeded rows, the first and last tiles, and both sides of every 2048-token
    # boundary (the transform / correction overlap splits the tokens there)
    edges = [e for b in range(2048, w.tokens, 2048) for e in (b - 1, b)]
    rows = np.unique(np.concatenate([np.random.default_rng(3).choice(w.tokens, size=24, replace=False),
                                     [0, 63, 64, w.tokens - 1], edges]))
    check_contract(w, codes, scales, zeros, rot, rows=rows, label=f"{name} rows {len(rows)}")
    # without the rotated output (the other correction kernel): identical outputs
    x, v, wt = to_dev_bf16(w.x), to_dev_f32(w.v), to_dev_f32(w.w_t)
    c2, s2, z2 = ops.rotate_quant(x, hadamard=w.hadamard, v=v, w_t=wt, rank_block=w.rank_block, group=w.group)
    torch.cuda.synchronize()
    assert np.array_equal(c2.cpu().numpy(), codes)
    assert np.array_equal(f16_bits(s2), scales) and np.array_equal(f16_bits(z2), zeros)


def test_prepared_factors_give_identical_outputs():
    print("[test_prepared_factors_give_identical_outputs]", flush=True)
    w = SMALL["downproj_8b"]()
    prep = ops.prepare_rank_factors(to_dev_f32(w.v), to_dev_f32(w.w_t), w.n, w.k)
    a = run_mfma(w)
    b = run_mfma(w, prepared=prep)
    for p, q in zip(a, b):
        assert np.array_equal(p, q)


def test_kronecker_hadamard_only_mfma():
    """k = 0: the Paley product on MFMA against the oracle's fp64 definition."""
    print("[test_kronecker_hadamard_only_mfma]", flush=True)
    for make in (lambda: workloads.downproj_8b(tokens=64), lambda: workloads.qproj_3b(tokens=64)):
        w = make()
        w.v = w.w_t = None
        x = to_dev_bf16(w.x)
        rot = torch.empty((w.tokens, w.n), dtype=torch.float32, device="cuda")
        codes, scales, zeros = ops.rotate_quant(x, hadamard=w.hadamard, group=w.group, rotated=rot)
        torch.cuda.synchronize()
        ref_rot, ref = oracle_for(w)
        rot = rot.cpu().numpy()
        frac_exact = float((rot == ref_rot).mean())
        print(f"  {w.name}: rotated bit-exact fraction {frac_exact:.6f}, err {O.rotated_error(rot, ref_rot):.3e}")
        # P = fma(hm, S1, hm*S23) rounds hm*S23 first: a 1-ulp difference from the
        # correctly rounded value where hm*S lies within 2^-33|P| of a midpoint
        # (about 2^-8 of the elements)
        assert frac_exact > 0.99
        assert O.rotated_error(rot, ref_rot) <= 2.0 ** -23
        rep = O.compare_quant(ref_rot, ref, O.unpack(codes.cpu().numpy(), w.n), f16_bits(scales), f16_bits(zeros),
                              w.group, rel_err=2.0 ** -23)
        assert rep.within_contract(), rep


def test_block_hadamard_full_row_rank_mfma():
    """E17 shape: block-H_128 over an 8B down_proj row with a k=32 full-row rank."""
    print("[test_block_hadamard_full_row_rank_mfma]", flush=True)
    w = workloads.downproj_8b(tokens=80)
    w.hadamard = (1, 128)
    check_contract(w, *run_mfma(w), label="blockH128 k32")


def test_projection_mfma_close_to_exact():
    print("[test_projection_mfma_close_to_exact]", flush=True)
    w = SMALL["downproj_8b"]()
    x = to_dev_bf16(w.x)
    v = to_dev_f32(w.v)
    prep = ops.prepare_rank_factors(v, to_dev_f32(w.w_t), w.n, w.k)
    p_m = torch.empty((w.tokens, 8 * w.k), dtype=torch.float32, device="cuda")
    ops.rank_projection(x, None, p_m, ops.RANK_MFMA, prepared=prep, k=w.k)
    torch.cuda.synchronize()
    u_m = p_m.cpu().numpy().reshape(w.tokens, 8, w.k).astype(np.float64).sum(axis=1)
    u_ref = O.projection(O.bf16_to_f32(w.x), w.v).astype(np.float64)
    rel = np.abs(u_m - u_ref) / (np.abs(u_ref) + np.sqrt((u_ref ** 2).mean()))
    print(f"  projection max rel err {rel.max():.3e}")
    assert rel.max() < 2.0 ** -20


def _zero_producing_rows(n: int, t: int) -> np.ndarray:
    """Rows whose FWHT outputs contain exact zeros (zero and constant rows, a
    rounding-boundary ramp, a common offset, an outlier on noise) interleaved
    with plain noise rows, so that waves with and without a zero both occur."""
    rng = np.random.default_rng(29)
    noise = rng.standard_normal((t, n)).astype(np.float32)
    rows = noise.copy()
    rows[0] = 0.0
    rows[2] = 0.5
    rows[4] = ((np.arange(n) % 15 - 7 + 0.5) / 7).astype(np.float32)
    rows[6] = 64 + noise[6] * 0.03125
    rows[8, 0] = 128.0
    rows[9, : n // 2] = 0.0
    return O.bf16_bits(rows)


@pytest.mark.parametrize("shape", [(12, 256, 3072, 64), (28, 512, 14336, 128), (28, 1024, 28672, 128)])
def test_kron_mfma_zero_results_keep_ieee_sign(shape):
    """The Kronecker kernel's cross-lane butterflies run in a sign-folded form
    that is bit-exact for every nonzero value; a wave holding an exact zero (or a
    value below 2^-100) recomputes with the plain butterflies.  Rows that make
    zeros must therefore give the oracle's zero signs in the rotated rows and the
    oracle's fp16 zero-point bits (fp16(-0) would differ), k = 0 on the MFMA path."""
    m, q, n, b = shape
    print(f"[test_kron_mfma_zero_results_keep_ieee_sign] {shape}", flush=True)
    t = 12
    bits = _zero_producing_rows(n, t)
    x = to_dev_bf16(bits)
    rot = torch.empty((t, n), dtype=torch.float32, device="cuda")
    codes, scales, zeros = ops.rotate_quant(x, hadamard=(m, q), group=b, rotated=rot)
    torch.cuda.synchronize()
    ref_rot = O.rotate(O.bf16_to_f32(bits), m, q)
    ref = O.quant(ref_rot, b)
    rot = rot.cpu().numpy()
    z = ref_rot == 0
    assert z.any()
    # where the oracle is zero the kernel gives the same zero, or (MFMA class) a
    # residual of the split Paley sums far below the tolerance
    both = z & (rot == 0)
    assert both.sum() >= 0.99 * z.sum()
    assert np.array_equal(np.signbit(rot[both]), np.signbit(ref_rot[both]))
    assert O.rotated_error(rot, ref_rot) <= 2.0 ** -23
    assert np.array_equal(f16_bits(zeros), ref.zeros)
    rep = O.compare_quant(ref_rot, ref, O.unpack(codes.cpu().numpy(), n), f16_bits(scales), f16_bits(zeros), b,
                          rel_err=2.0 ** -23)
    assert rep.within_contract(), rep
