"""Host logic of the drop-in modules (no GPU): split heuristics, layouts,
config objects, factor-term helpers and the fp32 reference_transform."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O


def test_split_count_matches_reference_rule():
    from nar.kernels import r4_fused_v2 as k2
    assert k2.split_count(8192, 14336) == 1            # 1024 tiles >= 512
    assert k2.split_count(2048, 14336) == 2            # 256 tiles -> 2
    assert k2.split_count(64, 8192) == 32              # capped at MAX_SPLITS
    assert k2.split_count(1, 14336, override=7) == 7
    with pytest.raises(ValueError):
        k2.split_count(1, 14336, override=5)


def test_allocation_layouts():
    from nar.kernels import r4_fused_v2 as k2
    out = k2.allocate_outputs(3, 1024, torch.device("cpu"))
    assert out.codes.shape == (3, 512) and out.codes.dtype == torch.uint8
    assert out.scales.shape == (3, 8) and out.scales.dtype == torch.float16
    assert k2.allocate_outputs(3, 1024, torch.device("cpu"), group=32).scales.shape == (3, 32)
    with pytest.raises(ValueError):
        k2.allocate_outputs(3, 1000, torch.device("cpu"))
    assert k2.allocate_partial(5, 32, 4, torch.device("cpu")).shape == (5, 128)


def test_unpack_low_nibble_is_even_channel():
    from nar.kernels import r4_fused_v2 as k2
    codes = torch.tensor([[0x21, 0xF0]], dtype=torch.uint8)
    assert k2.unpack(codes, 4).tolist() == [[1, 2, 0, 15]]
    assert np.array_equal(O.unpack(codes.numpy(), 4), k2.unpack(codes, 4).numpy())


def test_v3_configs_and_padded_rank():
    from nar.kernels import r4_fused_v3 as k3
    assert [k3.padded_rank(k) for k in (1, 8, 16, 17, 32, 64)] == [16, 16, 16, 32, 32, 64]
    assert len(k3.PROJECTION_CONFIGS) == 24 and len(k3.TILE_CONFIGS) == 12
    assert k3.ProjectionConfig(16, 64, 2, 4, 4).label() == "T16_D64_S2_w4_s4"
    assert k3.TileConfig(16, 8, 3, True).label() == "T16_w8_s3_dot"


def test_v3_factor_terms_reconstruct_exactly():
    from nar.kernels import r4_fused_v3 as k3
    rng = np.random.default_rng(0)
    n, k = 256, 8
    y = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32) / 16)
    hi = y.to(torch.bfloat16)
    lo = (y - hi.float()).to(torch.bfloat16)
    third = (y - hi.float() - lo.float()).to(torch.bfloat16)
    kp = k3.padded_rank(k)
    terms = torch.zeros((3, n, kp), dtype=torch.bfloat16)
    terms[0, :, :k], terms[1, :, :k], terms[2, :, :k] = hi, lo, third
    v = k3._factor_from_terms(terms.reshape(3 * n, kp), n, k, 3)
    assert torch.equal(v, y)


def test_e28_helpers():
    import nar_r4_kernel as nk
    h = nk.sylvester_hadamard_fp16(torch.device("cpu")).float()
    i = torch.arange(128)
    pop = torch.tensor([[bin(int(a) & int(b)).count("1") for b in i] for a in i])
    assert torch.equal(h, (1 - 2 * (pop % 2)).float())
    rng = np.random.default_rng(1)
    w = torch.from_numpy(rng.standard_normal((8, 256)).astype(np.float32) / 16)
    hi, lo = nk.w_terms(w)
    assert (hi.float() + lo.float() - w).abs().max() <= 2.0 ** -22 * w.abs().max()
    y = torch.from_numpy(rng.standard_normal((256, 8)).astype(np.float32) / 16)
    terms = nk.fp16_terms(y, 8)
    assert terms.shape == (2 * 256, 16)
    x = torch.from_numpy(rng.standard_normal((4, 256)).astype(np.float32))
    got = nk.reference_transform(x, y, w).numpy()
    ref = O.rotate(x.numpy(), 1, 128, v=y.numpy(), wt=w.numpy())
    assert O.rotated_error(got, ref) < 1e-6
    row = nk.precision_row(torch.from_numpy(ref).half(), torch.from_numpy(ref))
    assert row["code_match_fraction"] > 0.99 and row["relative_l2"] < 1e-3


def test_e28_module_host_logic():
    import nar_r4_kernel as nk
    rng = np.random.default_rng(3)
    n, k = 1024, 8
    y = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32) / 32)
    w = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32) / 32)
    sel = {"1": {"proj": nk.PROJECTION_CONFIGS[0].__dict__, "tile": nk.REFERENCE_TILE.__dict__},
           "2048": {"proj": nk.PROJECTION_CONFIGS[0].__dict__, "tile": nk.TILE_CONFIGS[2].__dict__}}
    mod = nk.NARDownTransform(y, w, k, sel)
    assert mod.factor_bytes() == 2 * n * k * 4
    assert mod.plan(1500)[1] == nk.TILE_CONFIGS[2] and mod.plan(2)[1] == nk.REFERENCE_TILE
    # the reference's term buffers, built on demand for Kernel A / Kernel B harnesses
    assert mod.y_terms.shape == (2 * n, 16) and mod.w_hi.dtype == torch.float16
    assert mod.factor_bytes() == 2 * n * k * 4 + 2 * n * 16 * 2 + 2 * k * n * 2
    with pytest.raises(ValueError):
        mod(torch.zeros((2, n), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        mod(torch.zeros((2, n), dtype=torch.float16))          # host tensor
    with pytest.raises(ValueError):
        nk.NARDownTransform(torch.zeros((n, 72)), torch.zeros((72, n)), 72, sel)
    with pytest.raises(ValueError):
        nk.NARDownTransform(y, w[:, :512], k, sel)
