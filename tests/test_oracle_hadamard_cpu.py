"""The oracle's Hadamard constructions beyond the Llama widths, pinned to the
reference: the Qwen3 Paley factors (orders 20, 68, 76, 200) and
full_hadamard_rows on power-of-two rows of 2048-8192 channels and on
20 * 2^j, 76 * 2^j and 68 * 2^j rows (golden vectors written from the
reference by tests/golden/make_hadamard_vectors.py).

Pins: the +-1 patterns equal the reference's; H H^T = m I; the power-of-two
rows are the reference's fp32 FWHT bit for bit (its stage order is pinned);
the Paley rows agree with the reference's BLAS product to the rounding of
one fp32 sum (the oracle's fp64-sum-rounded-once definition).  Planted
mistakes (a transposed Paley II block, the fp32 scale where the reference
uses the fp64 one) fail.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "hadamard_vectors.npz")
ORDERS = (20, 68, 76, 200)


def _dispatch(n: int) -> tuple[int, int]:
    """full_hadamard_rows' order of constructions (nar/activation_experiments.py:188-217)."""
    for m in (28, 12):
        if n % m == 0 and (n // m) & (n // m - 1) == 0:
            return m, n // m
    if n & (n - 1):
        for m in ORDERS:
            if n % m == 0 and (n // m) & (n // m - 1) == 0:
                return m, n // m
    return 1, n


@pytest.mark.parametrize("m", ORDERS)
def test_paley_patterns_match_reference(m):
    h = O.paley(m).astype(np.int64)
    assert np.array_equal(h, GOLD[f"paley{m}_sign"].astype(np.int64))
    assert np.array_equal(h @ h.T, m * np.eye(m, dtype=np.int64))
    assert GOLD[f"paley{m}_scale"][0] == 1.0 / np.sqrt(np.float64(m))


def test_paley_ii_planted_transposed_block_fails():
    h = O.paley(76).astype(np.int64)
    bad = h.copy()
    bad[:38, 38:] = h[38:, :38].T * -1
    assert not np.array_equal(bad, GOLD["paley76_sign"].astype(np.int64))


def _cases():
    i = 0
    while f"fhr{i}_x" in GOLD:
        yield i
        i += 1


@pytest.mark.parametrize("i", list(_cases()))
def test_full_hadamard_rows_matches_reference(i):
    x, s, y = GOLD[f"fhr{i}_x"], GOLD[f"fhr{i}_s"], GOLD[f"fhr{i}_y"]
    n = x.shape[1]
    m, q = _dispatch(n)
    got = O.rotate(x, m, q, signs=s)
    if m == 1:
        assert np.array_equal(got, y), f"n={n}: FWHT differs from the reference's"
    else:
        # the reference's BLAS sum order is not pinned: within the fp32 rounding
        # of an m-term sum, relative to the sum of the terms' magnitudes
        f = O.rotate(x, 1, q, signs=s).reshape(-1, m, q).astype(np.float64)
        mag = np.einsum("ab,tbc->tac", np.abs(O.paley(m).astype(np.float64)) / np.sqrt(m), np.abs(f))
        err = np.abs(got.astype(np.float64) - y).reshape(mag.shape)
        assert np.all(err <= m * 2.0 ** -24 * mag + 1e-30), f"n={n}, m={m}: {np.max(err / (mag + 1e-30))}"
        # planted mistake: the transposed factor (Paley I is not symmetric) breaks the bound
        if not np.array_equal(O.paley(m), O.paley(m).T):
            ht = O.paley(m).T.astype(np.float64) / np.sqrt(m)
            wrong = np.einsum("ab,tbc->tac", ht, f).astype(np.float32).reshape(y.shape)
            bad = np.abs(wrong.astype(np.float64) - y).reshape(mag.shape)
            assert np.any(bad > m * 2.0 ** -24 * mag + 1e-30)


def test_fp64_scale_is_what_the_reference_uses_for_68():
    """For order 68 the reference forms the Paley product in fp64 with the fp64
    1/sqrt(68); the fp32 scale (the 12/28 convention) gives different rows."""
    idx = [i for i in _cases() if GOLD[f"fhr{i}_x"].shape[1] == 17408][0]
    x, s, y = GOLD[f"fhr{idx}_x"], GOLD[f"fhr{idx}_s"], GOLD[f"fhr{idx}_y"]
    f = O.rotate(x, 1, 256, signs=s).reshape(-1, 68, 256)
    h = O.paley(68).astype(np.float64)
    scale32 = np.float64(np.float32(1.0) / np.float32(np.sqrt(68.0)))
    wrong = np.einsum("ab,tbc->tac", h * scale32, f.astype(np.float64)).astype(np.float32).reshape(y.shape)
    right = np.einsum("ab,tbc->tac", h / np.sqrt(68.0), f.astype(np.float64)).astype(np.float32).reshape(y.shape)
    assert np.mean(right == y) > 0.99
    assert np.mean(wrong == y) < 0.9
