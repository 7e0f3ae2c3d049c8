"""Factors made by the offline pipeline, fed to the GPU kernels.

The chain the reference runs before its online kernels: calibrated
reflectors and a permutation (RotationFactor, nar/fold_signed_permutation.py)
are folded into Y' and W'' (FoldedR4.from_factor), the signed permutation
Q = S P moves into gate/up, and the down_proj input the kernels see is Q x.
Here the factors come straight out of narhip.factor_pipeline and go, in the
layouts the pipeline writes, into

- the E17 v2 launcher (y_prime_t_fp32, w_h_t_fp32),
- the E17 v3 launcher (y_prime_pad_terms_bf16, the hi/lo/third bf16 split),
- E28's fp16 NARDownTransform (y_prime_fp32, w_h_t_fp32 as exported).

Each output is checked against the oracle on the same factors (the tie
contract for INT4, <= 1 fp16 ulp on <= 1e-4 of the elements for E28) and,
end to end, against the unfolded rotation RotationFactor.apply of the raw
rows (as e28_v2/verify.py:33-36 checks the fold direction).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

import nar_r4_kernel as nk  # noqa: E402
from nar.kernels import r4_fused_v2 as k2  # noqa: E402
from nar.kernels import r4_fused_v3 as k3  # noqa: E402
from narhip import factor_pipeline as fp  # noqa: E402

REL_ERR = 2.0 ** -21

# (n, reflectors, inactive ones): rank 8 at the 3B intermediate width, rank 32
# at the 8B width with two reflectors switched off by calibration
CASES = [(8192, 8, ()), (14336, 34, (5, 20))]


def calibrated(n: int, r: int, off: tuple[int, ...], seed: int) -> fp.RotationFactor:
    g = torch.Generator().manual_seed(seed)
    refl = torch.randn((r, n), generator=g)
    refl /= refl.norm(dim=1, keepdim=True)
    active = torch.ones(r, dtype=torch.bool)
    active[list(off)] = False
    return fp.RotationFactor(n, 128, refl, active, torch.randperm(n, generator=g),
                             torch.randperm(n, generator=g), 0.0)


def folded_case(n, r, off, layer=3):
    f = calibrated(n, r, off, seed=n + r)
    signs = fp.signs_for(n, layer, 20260902)
    folded = fp.FoldedR4.from_factor(f, signs)
    assert folded.rank == r - len(off)
    return f, signs, folded


def raw_rows(tokens: int, n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((tokens, n), generator=g)
    x[:, 11::613] *= 30.0
    return x


def bits_of(x_bf16: torch.Tensor) -> np.ndarray:
    return x_bf16.cpu().view(torch.int16).numpy().view(np.uint16)


def check_int4(out, x_bits, folded, n):
    v = folded.y_prime_fp32.numpy()
    wt = folded.w_h_t_fp32.numpy()
    rot = O.rotate(O.bf16_to_f32(x_bits), 1, 128, v=v, wt=wt)
    ref = O.quant(rot, 128)
    codes, s, z = out.codes.cpu().numpy(), f16_bits(out.scales), f16_bits(out.zeros)
    rep = O.compare_quant(rot, ref, O.unpack(codes, n), s, z, 128, rel_err=REL_ERR)
    print("  ", rep, flush=True)
    assert rep.within_contract(), rep
    return codes, s, z


def unfolded_agreement(codes, s, z, raw_f32, f, signs, n):
    """Dequantized kernel output vs the unfolded rotation of the raw rows."""
    deq = O.dequant(codes, s, z, n, 128)
    want = f.apply(raw_f32, signs).numpy()
    rel = float(np.linalg.norm(deq - want) / np.linalg.norm(want))
    ref_codes = O.unpack(O.quant(np.ascontiguousarray(want, np.float32), 128).packed, n)
    match = float((O.unpack(codes, n) == ref_codes).mean())
    print(f"   unfolded: relative L2 {rel:.3e}, code match {match:.6f}", flush=True)
    assert rel < 0.12          # INT4 at group 128: about 1/15 of a group's range
    assert match >= 0.999


@pytest.mark.parametrize("n,r,off", CASES)
def test_v2_with_pipeline_factors(n, r, off):
    print(f"[test_v2_with_pipeline_factors] n={n} r={r} off={off}", flush=True)
    f, signs, folded = folded_case(n, r, off)
    k = folded.rank
    raw = raw_rows(40, n, seed=n).to(torch.bfloat16)
    x = folded.q_unfolded(raw.float()).to(torch.bfloat16).contiguous()     # Q x: exact in bf16
    assert torch.equal(x.float(), folded.q_unfolded(raw.float()))
    xd = x.cuda()
    splits = k2.split_count(x.shape[0], n)
    partial = k2.allocate_partial(x.shape[0], k, splits, xd.device)
    out = k2.allocate_outputs(x.shape[0], n, xd.device)
    k2.launch_nar(xd, folded.y_prime_t_fp32.cuda(), folded.w_h_t_fp32.cuda(), out, partial)
    torch.cuda.synchronize()
    codes, s, z = check_int4(out, bits_of(x), folded, n)
    unfolded_agreement(codes, s, z, raw.float(), f, signs, n)


@pytest.mark.parametrize("n,r,off", CASES)
def test_v3_with_pipeline_terms(n, r, off):
    print(f"[test_v3_with_pipeline_terms] n={n} r={r} off={off}", flush=True)
    f, signs, folded = folded_case(n, r, off)
    k = folded.rank
    assert folded.y_prime_pad_terms_bf16.shape == (3 * n, k3.padded_rank(k))
    raw = raw_rows(48, n, seed=n + 1).to(torch.bfloat16)
    x = folded.q_unfolded(raw.float()).to(torch.bfloat16).contiguous()
    xd = x.cuda()
    cfg = k3.PROJECTION_CONFIGS[0]
    partial = k3.allocate_partial(x.shape[0], k, cfg.splits, xd.device)
    k3.launch_projection_dot(xd, folded.y_prime_pad_terms_bf16.cuda(), partial, k, cfg, 3)
    out = k3.allocate_outputs(x.shape[0], n, xd.device)
    k3.launch_nar(xd, folded.w_h_t_fp32.cuda(), out, partial, k, k3.TILE_CONFIGS[4])
    torch.cuda.synchronize()
    codes, s, z = check_int4(out, bits_of(x), folded, n)
    unfolded_agreement(codes, s, z, raw.float(), f, signs, n)


@pytest.mark.parametrize("n,r,off", CASES)
def test_e28_with_exported_factors(n, r, off, tmp_path):
    print(f"[test_e28_with_exported_factors] n={n} r={r} off={off}", flush=True)
    f, signs, folded = folded_case(n, r, off)
    k = folded.rank
    path = tmp_path / f"nar_factors_test_k{k}.pt"
    fp.export_e28([folded], path, model="test", seed=20260902)
    layer = nk.load_factors(path, torch.device("cpu"))["layers"][0]
    mod = nk.NARDownTransform(layer["y_prime_fp32"], layer["w_h_t_fp32"], k, {}).cuda()
    raw = raw_rows(33, n, seed=n + 2).half()
    x = folded.q_unfolded(raw.float()).half().contiguous()
    out = mod(x.cuda())
    torch.cuda.synchronize()
    ref = O.rotate(x.float().numpy(), 1, 128, v=folded.y_prime_fp32.numpy(), wt=folded.w_h_t_fp32.numpy())
    got = out.cpu().numpy().view(np.uint16).astype(np.int32)
    exp = ref.astype(np.float16).view(np.uint16).astype(np.int32)
    signed = lambda b: np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)  # noqa: E731
    d = np.abs(signed(got) - signed(exp))
    print(f"   max ulp {d.max()}, differing {(d != 0).mean():.2e}", flush=True)
    assert d.max() <= 1 and (d != 0).mean() <= 1e-4
    # the fold direction, as the reference's verify measures it
    old = f.apply(raw.float(), signs)
    rel = float((out.float().cpu() - old).norm() / old.norm())
    print(f"   unfolded vs kernel relative L2 {rel:.3e}", flush=True)
    assert rel <= 2e-3
