"""GPU drop-ins for the hook-side functions (narhip.hooks).

* dynamic_asym_int4 against the reference's own outputs: the 36 golden cases
  written from nar/experiment.py:dynamic_asym_int4 (zero, constant, rounding
  boundary, common offset, outlier, fp16-underflow hazard, near-constant,
  subnormal scale, huge values, ...), bit for bit: unpacked codes, fp16 scale
  and zero, fp32 dequantized values.  bf16 and fp16 inputs: the same against
  the oracle on the converted values, deq rounded to the input dtype.
* full_hadamard_rows against the oracle (which the golden full_hadamard_rows
  vectors pin on the CPU): bit-exact for block Hadamards; within 2^-21 of the
  row scale where the Paley factor runs on MFMA.
* rotate_dynamic_asym_int4 with a rank-k term: the oracle's tuple of x'.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from helpers import f16_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import hooks, workloads  # noqa: E402

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "reference_vectors.npz")
CASES = sorted({k.rsplit("_", 1)[0] for k in GOLD.files if k.startswith("q_") and k.endswith("_x")})


@pytest.mark.parametrize("case", CASES)
def test_dynamic_asym_int4_reference_vectors(case):
    b = int(case.rsplit("_b", 1)[1])
    x = GOLD[f"{case}_x"]
    deq, s, z, codes = hooks.dynamic_asym_int4(torch.from_numpy(x).cuda(), b)
    torch.cuda.synchronize()
    rows, n = x.shape
    assert codes.shape == (rows, n // b, b) and codes.dtype == torch.uint8
    assert s.shape == (rows, n // b) and s.dtype == torch.float16
    assert deq.shape == x.shape and deq.dtype == torch.float32
    assert np.array_equal(codes.cpu().numpy().reshape(rows, n), GOLD[f"{case}_codes"].reshape(rows, n))
    assert np.array_equal(f16_bits(s), GOLD[f"{case}_scale"].reshape(rows, n // b))
    assert np.array_equal(f16_bits(z), GOLD[f"{case}_zero"].reshape(rows, n // b))
    assert np.array_equal(deq.cpu().numpy().view(np.uint32), GOLD[f"{case}_deq"].reshape(rows, n).view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b", [32, 128])
def test_dynamic_asym_int4_half_inputs(dtype, b):
    print(f"[test_dynamic_asym_int4_half_inputs] {dtype} b={b}", flush=True)
    g = torch.Generator().manual_seed(7)
    x = (torch.randn((3, 5, 512), generator=g) * 3).to(dtype)
    deq, s, z, codes = hooks.dynamic_asym_int4(x.cuda(), b)
    torch.cuda.synchronize()
    xf = x.float().numpy().reshape(-1, 512)
    ref = O.quant(xf, b)
    assert deq.dtype == dtype and deq.shape == x.shape
    assert codes.shape == (3, 5, 512 // b, b)
    assert np.array_equal(codes.cpu().numpy().reshape(-1, 512), ref.codes)
    assert np.array_equal(f16_bits(s).reshape(-1, 512 // b), ref.scales)
    assert np.array_equal(f16_bits(z).reshape(-1, 512 // b), ref.zeros)
    want = torch.from_numpy(ref.deq).to(dtype).view(3, 5, 512)
    assert torch.equal(deq.cpu().view(torch.int16), want.view(torch.int16))


def test_dynamic_asym_int4_errors():
    with pytest.raises(ValueError, match="not divisible by group size"):
        hooks.dynamic_asym_int4(torch.zeros((2, 96), device="cuda"), 64)


@pytest.mark.parametrize("idx", [4, 5, 6, 7])
def test_full_hadamard_rows_vs_oracle(idx):
    print(f"[test_full_hadamard_rows_vs_oracle] fhr{idx}", flush=True)
    x = GOLD[f"fhr{idx}_x"]
    signs = GOLD[f"fhr{idx}_s"]
    xb = torch.from_numpy(x).bfloat16()
    out = hooks.full_hadamard_rows(xb.float().cuda(), torch.from_numpy(signs).cuda())
    torch.cuda.synchronize()
    n = x.shape[1]
    m, q = {3072: (12, 256), 14336: (28, 512), 128: (1, 128), 1024: (1, 1024)}[n]
    ref = O.rotate(xb.float().numpy(), m, q, signs=signs)
    obs = out.cpu().numpy()
    assert out.shape == x.shape and out.dtype == torch.float32
    if m == 1:
        assert np.array_equal(obs, ref)
    else:
        assert O.rotated_error(obs, ref) <= 2.0 ** -21


def test_full_hadamard_rows_inf_row_stays_in_its_row():
    """H28 x H1024 runs on the persistent Kronecker kernel (one workgroup per
    CU walks several tokens): an Inf in token 0 must not reach token 0 +
    grid through the zero-padded Paley rows in LDS."""
    print("[test_full_hadamard_rows_inf_row_stays_in_its_row] 600 x 28672", flush=True)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((600, 28 * 1024)).astype(np.float32)
    xb = torch.from_numpy(x).bfloat16()
    xb[0, 5] = float("inf")
    out = hooks.full_hadamard_rows(xb.float().cuda(), None)
    torch.cuda.synchronize()
    obs = out.cpu().numpy()
    ref = O.rotate(xb[1:].float().numpy(), 28, 1024)
    assert np.isfinite(obs[1:]).all()
    assert O.rotated_error(obs[1:], ref) <= 2.0 ** -21
    assert not np.isfinite(obs[0]).all()


def test_full_hadamard_rows_rejects_non_bf16_values():
    x = torch.full((2, 128), 1.0 + 2.0 ** -12, device="cuda")
    with pytest.raises(ValueError, match="bf16"):
        hooks.full_hadamard_rows(x, None)


def test_rotate_dynamic_asym_int4_with_rank():
    print("[test_rotate_dynamic_asym_int4_with_rank]", flush=True)
    w = workloads.qproj_3b(tokens=20)
    x = torch.from_numpy(O.bf16_to_f32(w.x)).view(4, 5, w.n)
    deq, s, z, codes = hooks.rotate_dynamic_asym_int4(
        x.cuda(), w.group, v=torch.from_numpy(w.v).cuda(), w_t=torch.from_numpy(w.w_t).cuda())
    torch.cuda.synchronize()
    ref_rot = O.rotate(O.bf16_to_f32(w.x), *w.hadamard, v=w.v, wt=w.w_t)
    ref = O.quant(ref_rot, w.group)
    G = w.n // w.group
    assert codes.shape == (4, 5, G, w.group) and s.shape == (4, 5, G) and deq.shape == (4, 5, w.n)
    rep = O.compare_quant(ref_rot, ref, codes.cpu().numpy().reshape(20, w.n), f16_bits(s).reshape(20, G),
                          f16_bits(z).reshape(20, G), w.group, rel_err=2.0 ** -21)
    assert rep.within_contract(), rep
