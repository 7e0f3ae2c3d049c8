"""The offline factor pipeline (narhip.factor_pipeline, nar.fold_signed_permutation).

Pinned three ways: golden vectors written from the reference's compact_wy,
FoldedR4 and RotationFactor.apply (tests/golden/make_factor_vectors.py), the
closed forms the construction fixes (prod (I - 2 v v^T) = I - W Y^T; the
folded row form equals the unfolded rotation on Q x; W'' columns are block
Hadamards, checked against the oracle's FWHT), and file round trips of the
reference's schemas (RotationFactor .pt, FoldedR4 payload, E28 export read by
nar_r4_kernel.load_factors).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

from narhip import factor_pipeline as fp  # noqa: E402

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "factor_vectors.npz")


def golden_factor() -> fp.RotationFactor:
    return fp.RotationFactor(n=256, b=128, reflectors=torch.from_numpy(GOLD["reflectors"]),
                             active=torch.from_numpy(GOLD["active"]),
                             source_order=torch.from_numpy(GOLD["source_order"]),
                             target_order=torch.from_numpy(GOLD["target_order"]), anchor_error=0.125)


def test_compact_wy_reference_vectors_and_closed_form():
    f = golden_factor()
    w, y = fp.compact_wy(f.reflectors, f.active)
    np.testing.assert_allclose(w.numpy(), GOLD["wy_w"], rtol=0, atol=2e-6)
    np.testing.assert_array_equal(y.numpy(), GOLD["wy_y"])
    # prod over active reflectors, in order, of (I - 2 v v^T) in fp64
    g = np.eye(256)
    for v, on in zip(GOLD["reflectors"].astype(np.float64), GOLD["active"]):
        if on:
            g = g @ (np.eye(256) - 2.0 * np.outer(v, v))
    np.testing.assert_allclose(np.eye(256) - w.double().numpy() @ y.double().numpy().T, g, atol=5e-6)
    # planted mistake: dropping the recurrence's cross term breaks the identity
    w_bad = 2.0 * y
    assert np.abs(np.eye(256) - w_bad.double().numpy() @ y.double().numpy().T - g).max() > 1e-2


def test_compact_wy_no_active_reflector():
    w, y = fp.compact_wy(torch.ones((2, 64)), torch.tensor([False, False]))
    assert w.shape == (64, 0) and y.shape == (64, 0)


def test_folded_factors_match_reference_vectors():
    f = golden_factor()
    signs = torch.from_numpy(GOLD["signs"])
    folded = fp.FoldedR4.from_factor(f, signs)
    assert folded.rank == 5
    np.testing.assert_array_equal(folded.source.numpy(), GOLD["source_for_target"])
    np.testing.assert_allclose(folded.y_prime_fp32.numpy(), GOLD["y_prime_fp32"], rtol=0, atol=2e-6)
    np.testing.assert_array_equal(folded.w_h_t_fp32.numpy(), GOLD["w_h_t_fp32"])
    np.testing.assert_array_equal(folded.w_h_fp32.numpy(), GOLD["w_h_fp32"])
    # bf16 terms: equal bits wherever Y' itself is bit-equal to the reference's
    same = folded.y_prime_fp32.numpy().view(np.uint32) == GOLD["y_prime_fp32"].view(np.uint32)
    terms = folded.y_prime_pad_terms_bf16.view(torch.int16).numpy().reshape(3, 256, 16)[:, :, :5]
    ref = GOLD["terms_bf16_bits"].reshape(3, 256, 16)[:, :, :5]
    assert same.mean() > 0.9
    assert np.array_equal(terms[:, same], ref[:, same])
    x = torch.from_numpy(GOLD["x"])
    np.testing.assert_array_equal(folded.q_unfolded(x).numpy(), GOLD["q_unfolded"])
    np.testing.assert_allclose(folded.apply(folded.q_unfolded(x)).numpy(), GOLD["folded_apply"], rtol=0,
                               atol=2e-5 * np.abs(GOLD["folded_apply"]).max())
    np.testing.assert_allclose(f.apply(x, signs).numpy(), GOLD["rotation_apply"], rtol=0,
                               atol=2e-5 * np.abs(GOLD["rotation_apply"]).max())


def test_fold_equals_unfolded_rotation():
    """H G' (Q x) = the unfolded rotation of x (the E17 v2 fold identity)."""
    g = torch.Generator().manual_seed(5)
    n, r = 512, 8
    refl = torch.randn((r, n), generator=g)
    refl /= refl.norm(dim=1, keepdim=True)
    f = fp.RotationFactor(n, 128, refl, torch.ones(r, dtype=torch.bool), torch.randperm(n, generator=g),
                          torch.randperm(n, generator=g), 0.0)
    signs = fp.signs_for(n, 3, 20260902)
    folded = fp.FoldedR4.from_factor(f, signs)
    x = torch.randn((7, n), generator=g)
    old = f.apply(x, signs)
    new = folded.apply(folded.q_unfolded(x))
    assert float((old - new).norm() / old.norm()) < 2e-6
    # W'' columns are FWHT_128 blocks of Q wy_y: equal to the oracle's transform
    w_prime = fp.signed_permute_rows(fp.compact_wy(refl, f.active)[1], folded.source, signs)
    ref = O.rotate(np.ascontiguousarray(w_prime.T.numpy()), 1, 128)
    np.testing.assert_array_equal(folded.w_h_t_fp32.numpy(), ref)


def test_signs_and_fold_into_swiglu():
    s = fp.signs_for(64, 2, 7)
    assert set(s.unique().tolist()) == {-1.0, 1.0} and torch.equal(s, fp.signs_for(64, 2, 7))
    g = torch.Generator().manual_seed(9)
    n, hidden = 256, 32
    refl = torch.randn((2, n), generator=g)
    refl /= refl.norm(dim=1, keepdim=True)
    f = fp.RotationFactor(n, 128, refl, torch.ones(2, dtype=torch.bool), torch.randperm(n, generator=g),
                          torch.randperm(n, generator=g), 0.0)
    folded = fp.FoldedR4.from_factor(f, fp.signs_for(n, 0, 1))
    gate, up = torch.nn.Linear(hidden, n, bias=False), torch.nn.Linear(hidden, n, bias=False)
    h = torch.randn((3, hidden), generator=g)
    before = torch.nn.functional.silu(gate(h)) * up(h)
    fp.fold_swiglu_weights(gate, up, folded)
    after = torch.nn.functional.silu(gate(h)) * up(h)
    torch.testing.assert_close(after, folded.q_unfolded(before), rtol=1e-6, atol=1e-6)
    with pytest.raises(AssertionError):
        fp.fold_swiglu_weights(torch.nn.Linear(hidden, n), up, folded)


def test_file_formats_round_trip(tmp_path):
    import nar_r4_kernel as nk
    f = golden_factor()
    f.save(tmp_path / "down_layer_00.pt", {"site": "down"})
    g = fp.RotationFactor.load(tmp_path / "down_layer_00.pt")
    assert g.n == 256 and g.b == 128 and g.anchor_error == 0.125
    assert torch.equal(g.reflectors, f.reflectors) and torch.equal(g.active, f.active)
    assert torch.equal(g.source_order, f.source_order) and torch.equal(g.target_order, f.target_order)
    folded = fp.FoldedR4.from_factor(g, torch.from_numpy(GOLD["signs"]))
    folded.save(tmp_path / "folded.pt", {"layer": 0})
    back = fp.FoldedR4.load(tmp_path / "folded.pt")
    for name in ("source", "signs", "y_prime_fp32", "w_h_t_fp32", "w_h_fp32", "y_prime_pad_terms_bf16"):
        assert torch.equal(getattr(back, name), getattr(folded, name)), name
    payload = fp.export_e28([folded, folded], tmp_path / "e28" / "nar_factors_x_k5.pt", model="x", seed=0)
    assert payload["rank"] == 5 and payload["group_size"] == 128
    loaded = nk.load_factors(tmp_path / "e28" / "nar_factors_x_k5.pt", torch.device("cpu"))
    assert len(loaded["layers"]) == 2
    assert torch.equal(loaded["layers"][1]["w_h_t_fp32"], folded.w_h_t_fp32)
    mod = nk.NARDownTransform(loaded["layers"][0]["y_prime_fp32"], loaded["layers"][0]["w_h_t_fp32"], 5, {})
    assert mod.factor_bytes() == 2 * 256 * 5 * 4


def test_drop_in_module_names():
    from nar import fold_signed_permutation as fsp
    for name in ("source_for_target", "signed_permute_rows", "block_hadamard_columns", "FoldedR4",
                 "fold_swiglu_weights", "precompute", "main"):
        assert hasattr(fsp, name), name
