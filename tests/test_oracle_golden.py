"""Pin the CPU oracle before trusting it.

Checks, by what fixes each part of the path:
  * golden vectors written from the reference's own functions
    (tests/golden/make_reference_vectors.py): Paley factors, full_hadamard_rows,
    _fast_walsh_hadamard, dynamic_asym_int4, reference_transform
  * the reference's E0 known answers (results/e0.json, seed 20260902)
  * closed forms: Sylvester H[i,j] = (-1)^popcount(i&j)/sqrt(q), H H = I,
    Paley H H^T = m I, the Kronecker product as a dense fp64 matrix
  * planted mistakes: a transposed Paley factor, a swapped Kronecker order, a
    multiply instead of a divide and a missing rank term must all fail.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD / "reference_vectors.npz")


def _factors(n):
    for m in (28, 12):
        q, r = divmod(n, m)
        if not r and not q & (q - 1):
            return m, q
    return 1, n


def _scaled_err(o, y):
    return O.rotated_error(o, y)


# ------------------------------------------------------------------ Paley ---

@pytest.mark.parametrize("m", [12, 28])
def test_paley_matches_reference_exactly(gold, m):
    ref = gold[f"paley{m}"]
    mine = O.paley(m).astype(np.float32) / np.float32(math.sqrt(m))
    assert np.array_equal(ref, mine)


@pytest.mark.parametrize("m", [12, 28])
def test_paley_is_hadamard(m):
    h = O.paley(m).astype(np.int64)
    assert np.array_equal(h @ h.T, m * np.eye(m, dtype=np.int64))
    assert (h[0] == 1).all() and (h[:, 0] == 1).all()


# ------------------------------------------------------------------- FWHT ---

@pytest.mark.parametrize("q", [32, 128, 512, 1024])
def test_fwht_bit_exact_with_reference(gold, q):
    assert np.array_equal(O.rotate(gold[f"fwht{q}_x"], 1, q), gold[f"fwht{q}_y"])


@pytest.mark.parametrize("q", [8, 64, 128, 256])
def test_fwht_closed_form_and_involution(q):
    i = np.arange(q)
    pop = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    h = ((-1.0) ** pop) / math.sqrt(q)
    x = np.random.default_rng(q).standard_normal((5, q)).astype(np.float32)
    y = O.rotate(x, 1, q)
    assert np.abs(y - x.astype(np.float64) @ h.T).max() < 1e-5 * np.abs(x).sum(axis=1).max()
    back = O.rotate(y, 1, q)
    assert np.abs(back - x).max() < 1e-5 * np.abs(x).max()


def test_fwht_divides_by_fp32_sqrt():
    """q=128: the normalisation is a division by fp32(sqrt(128)), not a multiply by
    0.0883883... (nar/extended_experiment.py:456 vs nar/kernels/r4_fused_v2.py:52)."""
    x = np.zeros((1, 128), np.float32)
    rng = np.random.default_rng(3)
    vals = rng.standard_normal(4096).astype(np.float32)
    div = vals / np.float32(math.sqrt(128))
    mul = vals * np.float32(0.08838834764831845)
    which = np.nonzero(div != mul)[0]
    assert which.size > 0
    x[0, 0] = vals[which[0]]            # one-hot: every output is +-x/sqrt(128)
    y = O.rotate(x, 1, 128)
    assert np.all(np.abs(y) == div[which[0]].__abs__())


# ------------------------------------------------- Kronecker / full rows ---

def test_full_hadamard_rows_matches_reference(gold):
    """Layout, orientation and dispatch of full_hadamard_rows; the Paley product is a
    BLAS sgemm in the reference, so agreement is to its rounding (a few fp32 ulp)."""
    for i in range(8):
        x, s, y = gold[f"fhr{i}_x"], gold[f"fhr{i}_s"], gold[f"fhr{i}_y"]
        m, q = _factors(x.shape[1])
        o = O.rotate(x, m, q, signs=s)
        if m == 1:
            assert np.array_equal(o, y)
        else:
            assert _scaled_err(o, y) < 1e-6, (i, _scaled_err(o, y))


def test_kronecker_dense_closed_form():
    for m, q in ((12, 16), (28, 8)):
        n = m * q
        pal = O.paley(m).astype(np.float64) / math.sqrt(m)
        i = np.arange(q)
        pop = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
        hq = ((-1.0) ** pop) / math.sqrt(q)
        dense = np.kron(pal, hq)
        x = np.random.default_rng(n).standard_normal((3, n)).astype(np.float32)
        y = O.rotate(x, m, q)
        assert np.abs(y - x.astype(np.float64) @ dense.T).max() < 1e-5 * np.abs(x).max() * math.sqrt(n)
        # orthogonal: norms preserved
        assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


def test_planted_mistakes_fail(gold):
    """A transposed Paley factor or swapped Kronecker order must be caught by the fixture."""
    x, s, y = gold["fhr1_x"], gold["fhr1_s"], gold["fhr1_y"]   # 28 x 8
    m, q = 28, 8
    pal = O.paley(m).astype(np.float64) / math.sqrt(m)
    i = np.arange(q)
    pop = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    hq = ((-1.0) ** pop) / math.sqrt(q)
    xs = x.astype(np.float64) * s
    good = xs @ np.kron(pal, hq).T
    assert _scaled_err(good.astype(np.float32), y) < 1e-6
    assert _scaled_err((xs @ np.kron(pal.T, hq).T).astype(np.float32), y) > 1e-2
    assert _scaled_err((xs @ np.kron(hq, pal).T).astype(np.float32), y) > 1e-2 if q == m else True


# ------------------------------------------------------------- rank-k -------

def test_reference_transform_matches(gold):
    for i in range(2):
        key = f"rt{i}_out"
        if key not in gold.files:
            pytest.skip("reference_transform fixture not written")
        x, yv, w = gold[f"rt{i}_x"], gold[f"rt{i}_y"], gold[f"rt{i}_w"]
        o = O.rotate(x, 1, 128, v=yv, wt=w)
        assert _scaled_err(o, gold[key]) < 1e-6
        # planted: the correction added instead of subtracted is caught
        wrong = O.rotate(x, 1, 128, v=yv, wt=-w)
        assert _scaled_err(wrong, gold[key]) > 1e-3


def test_rank_k_closed_form_and_zero_factors():
    rng = np.random.default_rng(5)
    n, k = 256, 8
    x = rng.standard_normal((4, n)).astype(np.float32)
    v = (rng.standard_normal((n, k)) / 16).astype(np.float32)
    w = (rng.standard_normal((k, n)) / 16).astype(np.float32)
    h = O.rotate(x, 1, 128)
    full = O.rotate(x, 1, 128, v=v, wt=w)
    ref = h.astype(np.float64) - (x.astype(np.float64) @ v) @ w
    assert np.abs(full - ref).max() < 1e-5
    assert np.array_equal(O.rotate(x, 1, 128, v=np.zeros_like(v), wt=np.zeros_like(w)), h)
    u = O.projection(x, v)
    assert np.abs(u - x.astype(np.float64) @ v).max() < 1e-6


def test_per_block_rank():
    rng = np.random.default_rng(9)
    heads, d, k = 4, 128, 2
    x = rng.standard_normal((3, heads * d)).astype(np.float32)
    v = rng.standard_normal((heads * d, k)).astype(np.float32) / 8
    w = rng.standard_normal((k, heads * d)).astype(np.float32) / 8
    got = O.rotate(x, 1, 128, v=v, wt=w, rank_block=d)
    h = O.rotate(x, 1, 128)
    for hd in range(heads):
        sl = slice(hd * d, (hd + 1) * d)
        u = x[:, sl].astype(np.float64) @ v[sl]
        assert np.abs(got[:, sl] - (h[:, sl] - u @ w[:, sl])).max() < 1e-5


# -------------------------------------------------------------- quantizer ---

def test_quantizer_bit_exact_with_reference(gold):
    names = list(gold["q_names"])
    assert len(names) >= 30
    for key in names:
        x = gold[key + "_x"]
        b = int(key.split("_b")[-1])
        r = O.quant(x, b)
        assert np.array_equal(r.codes, gold[key + "_codes"]), key
        assert np.array_equal(r.scales, gold[key + "_scale"]), key
        assert np.array_equal(r.zeros, gold[key + "_zero"]), key
        assert np.array_equal(r.deq, gold[key + "_deq"]), key


def test_e0_known_answers():
    """nar/experiment.py:329-384 on the reference's own seeds; values from results/e0.json."""
    torch = pytest.importorskip("torch")
    e0 = json.loads((GOLD / "e0_reference.json").read_text())
    seed = e0["seed"]
    for row in e0["rows"]:
        b = row["b"]
        if row["check"] == "constant_shift":
            g = torch.Generator().manual_seed(seed + b)
            x = torch.randn((512, b), generator=g, dtype=torch.float32).numpy()
            for shift, key_range, key_mse in ((0.0, "base_range", "base_mse"), (row["c"], "shifted_range", "shifted_mse")):
                xs = (x + np.float32(shift)).astype(np.float32)
                r = O.quant(xs, b)
                rng_mean = float((xs.max(axis=1) - xs.min(axis=1)).astype(np.float32).mean(dtype=np.float64))
                mse = float(((r.deq.astype(np.float64) - xs) ** 2).sum() / xs.size)
                assert abs(rng_mean - row[key_range]) <= 2e-6 * max(1.0, row[key_range])
                assert abs(mse - row[key_mse]) <= 1e-6 * row[key_mse], (b, shift, mse, row[key_mse])
        else:
            x = np.zeros((1, b), np.float32)
            x[0, 1] = row["amplitude"]
            y = O.rotate(x, 1, b)
            assert float(y.max() - y.min()) == pytest.approx(row["hadamard_range"], abs=0, rel=0)


def test_quantizer_round_half_even_at_exact_ties():
    """(x - z)/s exactly k + 1/2 rounds to even (torch.round, nar/experiment.py:182);
    the Triton kernel's floor(q + 0.5) (nar/kernels/r4_fused_v2.py:78) would not."""
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [0.0, 15.0, 2.5, 3.5, 0.5, 14.5]
    r = O.quant(x, 32)
    assert O.f16_bits_to_f32(r.scales)[0, 0] == 1.0 and O.f16_bits_to_f32(r.zeros)[0, 0] == 0.0
    assert list(r.codes[0, :6]) == [0, 15, 2, 4, 0, 14]
    floor_half = np.floor(x[0, :6] + np.float32(0.5))
    assert list(floor_half) != list(r.codes[0, :6])


def test_fp16_conversion_matches_numpy():
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000).astype(np.float32),
        np.array([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 6.1e-5, -0.0, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    lib = O.lib()
    mine = np.array([lib.nar_oracle_f32_to_f16(float(v)) for v in vals[:20000]], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, want[:20000])
    tail = np.array([lib.nar_oracle_f32_to_f16(float(v)) for v in vals[-11:]], np.uint16)
    assert np.array_equal(tail, want[-11:])


def test_comparator_classifies_ties():
    """A 1-ulp perturbation of x' yields only explained mismatches; a gross one does not."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    ref = O.quant(x, 128)
    bumped = np.nextafter(x, np.float32(np.inf)).astype(np.float32)
    obs = O.quant(bumped, 128)
    rep = O.compare_quant(x, ref, obs.codes, obs.scales, obs.zeros, 128, rel_err=2.0 ** -22)
    assert rep.code_mismatch_unexplained == 0 and rep.scale_mismatch_unexplained == 0
    gross = O.quant(x * np.float32(1.001), 128)
    rep2 = O.compare_quant(x, ref, gross.codes, gross.scales, gross.zeros, 128, rel_err=2.0 ** -22)
    assert not rep2.within_contract()


def test_quantizer_nonfinite_groups_match_reference():
    """Groups holding NaN or +-Inf (tests/golden/make_nonfinite_vectors.py, written
    from nar/experiment.py:dynamic_asym_int4): NaN wins the group min/max
    (torch.amin/amax), the zero-point is the canonical quiet NaN, codes of NaN
    quotients are 0 and their dequantized values NaN."""
    nf = np.load(GOLD / "nonfinite_vectors.npz")
    names = list(nf["nf_names"])
    assert len(names) >= 27
    for key in names:
        x = nf[key + "_x"]
        b = int(key.split("_b")[-1])
        with np.errstate(invalid="ignore", over="ignore"):
            r = O.quant(x, b)
        assert np.array_equal(r.codes, nf[key + "_codes"]), key
        assert np.array_equal(r.scales, nf[key + "_scale"]), key
        assert np.array_equal(r.zeros, nf[key + "_zero"]), key
        assert np.array_equal(r.deq, nf[key + "_deq"], equal_nan=True), key


def test_quantizer_nonfinite_planted_mistake_fails():
    """Dequantizing the integer code (0 * 1 + Inf = Inf) instead of the NaN
    quotient must disagree with the reference on an all-Inf group."""
    nf = np.load(GOLD / "nonfinite_vectors.npz")
    key = "nf_all_inf_b32"
    r = O.quant(nf[key + "_x"], 32)
    codes = r.codes.astype(np.float32).reshape(r.deq.shape)
    s = O.f16_bits_to_f32(r.scales).repeat(32, axis=1)
    z = O.f16_bits_to_f32(r.zeros).repeat(32, axis=1)
    with np.errstate(invalid="ignore"):
        wrong = codes * s + z
    assert not np.array_equal(wrong, nf[key + "_deq"], equal_nan=True)
