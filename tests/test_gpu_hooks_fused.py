"""The fused hook path (narhip.hooks.rotate_dynamic_asym_int4) and the wider
full_hadamard_rows domain against the oracle.

* One kernel per call (x read once) for the per-head forms of the K and V
  cache shapes (H_128 per head, per-head rank k = 2 and 4, groups of 32): the
  tuple (unpacked codes, fp16 scale and zero, fp32 deq) is the oracle's bit
  for bit, on all 2048 and 64 rows.
* The power-of-two rows of 2048, 4096 and 8192 channels (one FWHT over the
  row): full_hadamard_rows equals the oracle (pinned to the reference's
  vectors on the CPU) bit for bit, on the reference's own golden rows and on
  seeded rows, and the fused tuple too, at groups of 32 and 128.
* H_20 (x) H_128 / H_256 (the Qwen3 widths 2560 and 5120) and the Llama
  Kronecker widths without a rank term: full_hadamard_rows within 2^-21 of
  the row scale of the oracle (the Paley product runs on MFMA), the tuple
  within the tie contract.
* The two-kernel fallback (full-row rank, or a group the one-pass kernels do
  not build): the oracle's tuple bit for bit in exact rank mode.
* rotate_quant's packed output on the new widths, bit for bit.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from helpers import f16_bits, to_dev_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from narhip import hooks, ops, workloads  # noqa: E402

HGOLD = np.load(Path(__file__).resolve().parent / "golden" / "hadamard_vectors.npz")


def _tuple_np(res):
    deq, s, z, codes = res
    T = deq.reshape(-1, deq.shape[-1]).shape[0]
    n = deq.shape[-1]
    return (deq.cpu().numpy().reshape(T, n), f16_bits(s).reshape(T, -1), f16_bits(z).reshape(T, -1),
            codes.cpu().numpy().reshape(T, n))


def _assert_tuple_exact(got, ref, what):
    deq, s, z, codes = got
    assert np.array_equal(codes, ref.codes), f"{what}: codes"
    assert np.array_equal(s, ref.scales), f"{what}: scales"
    assert np.array_equal(z, ref.zeros), f"{what}: zeros"
    same = (deq.view(np.uint32) == ref.deq.view(np.uint32)) | (np.isnan(deq) & np.isnan(ref.deq))
    assert same.all(), f"{what}: deq"


def _seeded_bf16(rows, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, n)).astype(np.float32) * rng.choice([0.02, 1.0, 25.0], size=(rows, 1))
    x[:, rng.choice(n, size=6, replace=False)] *= np.float32(40.0)
    return workloads.bf16_bits(x.astype(np.float32))


@pytest.mark.parametrize("name", ["kcache_3b", "vcache_decode_8b"])
def test_fused_per_head_tuple_exact(name):
    w = workloads.CONFIGS[name]()
    print(f"[test_fused_per_head_tuple_exact] {name}: {w.tokens} x {w.n}, k={w.k} per head, b={w.group}",
          flush=True)
    x = to_dev_bf16(w.x)
    v, wt = torch.from_numpy(w.v).cuda(), torch.from_numpy(w.w_t).cuda()
    res = hooks.rotate_dynamic_asym_int4(x, w.group, v=v, w_t=wt, block=128, rank_block=128)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(w.x), 1, 128, v=w.v, wt=w.w_t, rank_block=128), w.group)
    _assert_tuple_exact(_tuple_np(res), ref, name)


def test_fused_per_head_leading_dims_and_signs():
    """[batch, tokens, heads * head_dim] input with signs: shapes follow the reference's tuple."""
    w = workloads.kcache_3b(48)
    signs = np.where(np.arange(w.n) % 5 == 0, -1.0, 1.0).astype(np.float32)
    x = to_dev_bf16(w.x).view(4, 12, w.n)
    res = hooks.rotate_dynamic_asym_int4(x, 32, signs=torch.from_numpy(signs).cuda(),
                                         v=torch.from_numpy(w.v).cuda(), w_t=torch.from_numpy(w.w_t).cuda(),
                                         block=128, rank_block=128)
    torch.cuda.synchronize()
    deq, s, z, codes = res
    assert deq.shape == (4, 12, w.n) and s.shape == (4, 12, w.n // 32) and codes.shape == (4, 12, w.n // 32, 32)
    ref = O.quant(O.rotate(O.bf16_to_f32(w.x), 1, 128, signs=signs, v=w.v, wt=w.w_t, rank_block=128), 32)
    _assert_tuple_exact(_tuple_np(res), ref, "kcache [4, 12, 1024] with signs")


def _golden_rows(n):
    for i in range(16):
        if f"fhr{i}_x" not in HGOLD:
            break
        if HGOLD[f"fhr{i}_x"].shape[1] == n:
            return HGOLD[f"fhr{i}_x"], HGOLD[f"fhr{i}_s"], HGOLD[f"fhr{i}_y"]
    raise KeyError(n)


@pytest.mark.parametrize("n", [2048, 4096, 8192])
def test_full_hadamard_rows_power_of_two_rows(n):
    print(f"[test_full_hadamard_rows_power_of_two_rows] n={n}", flush=True)
    x, s, y = _golden_rows(n)
    out = hooks.full_hadamard_rows(torch.from_numpy(x).cuda(), torch.from_numpy(s).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), y), "differs from the reference's own rows"
    bits = _seeded_bf16(37, n, n)
    out = hooks.full_hadamard_rows(to_dev_bf16(bits), None)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.rotate(O.bf16_to_f32(bits), 1, n))


@pytest.mark.parametrize("n", [2048, 4096, 8192])
@pytest.mark.parametrize("b", [32, 128])
def test_fused_power_of_two_tuple_exact(n, b):
    print(f"[test_fused_power_of_two_tuple_exact] n={n} b={b}", flush=True)
    bits = _seeded_bf16(70, n, 3 * n + b)
    signs = np.where(np.arange(n) % 3 == 1, -1.0, 1.0).astype(np.float32)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(bits), b, signs=torch.from_numpy(signs).cuda())
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(bits), 1, n, signs=signs), b)
    _assert_tuple_exact(_tuple_np(res), ref, f"n={n} b={b}")


@pytest.mark.parametrize("n", [4096, 8192])
def test_rotate_quant_packed_power_of_two(n):
    bits = _seeded_bf16(33, n, n + 1)
    codes, s, z = ops.rotate_quant(to_dev_bf16(bits), hadamard=(1, n), group=128)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(bits), 1, n), 128)
    assert np.array_equal(codes.cpu().numpy(), ref.packed)
    assert np.array_equal(f16_bits(s), ref.scales) and np.array_equal(f16_bits(z), ref.zeros)


@pytest.mark.parametrize("n", [2560, 5120])
def test_full_hadamard_rows_paley20(n):
    print(f"[test_full_hadamard_rows_paley20] n={n}", flush=True)
    x, s, _ = _golden_rows(n)
    m, q = 20, n // 20
    out = hooks.full_hadamard_rows(torch.from_numpy(x).cuda(), torch.from_numpy(s).cuda())
    torch.cuda.synchronize()
    ref = O.rotate(x, m, q, signs=s)
    assert O.rotated_error(out.cpu().numpy(), ref) <= 2.0 ** -21
    bits = _seeded_bf16(40, n, n + 7)
    out = hooks.full_hadamard_rows(to_dev_bf16(bits), None)
    torch.cuda.synchronize()
    assert O.rotated_error(out.cpu().numpy(), O.rotate(O.bf16_to_f32(bits), m, q)) <= 2.0 ** -21


@pytest.mark.parametrize("n,m", [(9728, 76), (17408, 68)])
def test_full_hadamard_rows_large_paley_golden(n, m):
    """The Qwen3 widths 76 x 128 and 68 x 256 on the reference's own rows: the
    oracle's arithmetic exactly, and the reference's output within the fp32
    rounding of an m-term sum (its BLAS order is not pinned)."""
    print(f"[test_full_hadamard_rows_large_paley_golden] n={n} m={m}", flush=True)
    x, s, y = _golden_rows(n)
    q = n // m
    out = hooks.full_hadamard_rows(torch.from_numpy(x).cuda(), torch.from_numpy(s).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got, O.rotate(x, m, q, signs=s))
    f = O.rotate(x, 1, q, signs=s).reshape(-1, m, q).astype(np.float64)
    mag = np.einsum("ab,tbc->tac", np.abs(O.paley(m).astype(np.float64)) / np.sqrt(m), np.abs(f))
    err = np.abs(got.astype(np.float64) - y).reshape(mag.shape)
    assert np.all(err <= m * 2.0 ** -24 * mag + 1e-30)


@pytest.mark.parametrize("n,m,tokens", [(25600, 200, 5), (9728, 76, 33), (17408, 68, 3), (200 * 64, 200, 2)])
def test_full_hadamard_rows_large_paley_seeded(n, m, tokens):
    """Seeded bf16 rows (no golden rows of 200 x 128 exist), with and without
    signs, bit-equal to the oracle; zero rows stay zero."""
    print(f"[test_full_hadamard_rows_large_paley_seeded] n={n} m={m} tokens={tokens}", flush=True)
    q = n // m
    bits = _seeded_bf16(tokens, n, 3 * n + m)
    bits[0] = 0
    g = np.random.default_rng(n + 1)
    s = np.where(g.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    out = hooks.full_hadamard_rows(to_dev_bf16(bits), torch.from_numpy(s).cuda())
    torch.cuda.synchronize()
    ref = O.rotate(O.bf16_to_f32(bits), m, q, signs=s)
    assert np.array_equal(out.cpu().numpy(), ref)
    assert not out[0].any()
    out = hooks.full_hadamard_rows(to_dev_bf16(bits[1:]), None)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.rotate(O.bf16_to_f32(bits[1:]), m, q))


@pytest.mark.parametrize("n,m,group", [(9728, 76, 128), (25600, 200, 64)])
def test_fused_tuple_large_paley(n, m, group):
    """The hooks' rotate_dynamic_asym_int4 on the Qwen3 widths: x' staged, then the quantizer, bit-exact."""
    print(f"[test_fused_tuple_large_paley] n={n} m={m} group={group}", flush=True)
    bits = _seeded_bf16(6, n, 5 * n + group)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(bits), group)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(bits), m, n // m), group)
    _assert_tuple_exact(_tuple_np(res), ref, f"n={n} m={m} group={group}")


@pytest.mark.parametrize("n,m,q", [(2560, 20, 128), (5120, 20, 256), (3072, 12, 256), (14336, 28, 512)])
def test_fused_kronecker_tuple_contract(n, m, q):
    print(f"[test_fused_kronecker_tuple_contract] n={n}", flush=True)
    bits = _seeded_bf16(64, n, 11 * n)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(bits), 128)
    torch.cuda.synchronize()
    deq, s, z, codes = _tuple_np(res)
    rot = O.rotate(O.bf16_to_f32(bits), m, q)
    ref = O.quant(rot, 128)
    rep = O.compare_quant(rot, ref, codes, s, z, 128, rel_err=2.0 ** -21)
    assert rep.within_contract(), rep
    # deq follows the returned codes, scales and zeros exactly
    sf = O.f16_bits_to_f32(s).repeat(128, axis=1)
    zf = O.f16_bits_to_f32(z).repeat(128, axis=1)
    want = (codes.astype(np.float32) * sf).astype(np.float32) + zf
    assert np.array_equal(deq, want.astype(np.float32))


def test_fused_fallback_full_row_rank_exact():
    """Full-row rank (two kernels: x' staged, then the hooks' quantizer), exact rank mode."""
    w = workloads.e17_8b(tokens=40, k=8)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(w.x), 64, v=torch.from_numpy(w.v).cuda(),
                                         w_t=torch.from_numpy(w.w_t).cuda(), block=128,
                                         rank_mode=ops.RANK_EXACT)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(w.x), 1, 128, v=w.v, wt=w.w_t), 64)
    _assert_tuple_exact(_tuple_np(res), ref, "e17 k=8 full-row rank, exact")


def test_fused_fallback_group_16():
    w = workloads.kcache_3b(64)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(w.x), 16, v=torch.from_numpy(w.v).cuda(),
                                         w_t=torch.from_numpy(w.w_t).cuda(), block=128, rank_block=128)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(w.x), 1, 128, v=w.v, wt=w.w_t, rank_block=128), 16)
    _assert_tuple_exact(_tuple_np(res), ref, "kcache group 16")


def test_fused_nonfinite_rows():
    """NaN and +-Inf inside groups of the fused per-head path: the reference's tuple
    (NaN zero-point and deq for a NaN group; Inf handling of dynamic_asym_int4)."""
    w = workloads.kcache_3b(16)
    x = O.bf16_to_f32(w.x).copy()
    x[1, 5] = np.nan
    x[3, 200] = np.inf
    x[4, 300] = -np.inf
    x[6, 40:42] = [np.inf, -np.inf]
    bits = workloads.bf16_bits(x)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(bits), 32, block=128)
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(bits), 1, 128), 32)
    _assert_tuple_exact(_tuple_np(res), ref, "non-finite rows")


@pytest.mark.parametrize("n,m,k,tokens,group", [(9728, 76, 8, 21, 128), (17408, 68, 32, 3, 64), (25600, 200, 16, 2, 128)])
def test_fused_tuple_large_paley_rank(n, m, k, tokens, group):
    """RotationFactor.apply-style x' = H x - (x V) W''^T on the Qwen3 widths, then
    dynamic_asym_int4: exact projection and correction, bit-exact tuple."""
    print(f"[test_fused_tuple_large_paley_rank] n={n} m={m} k={k} tokens={tokens}", flush=True)
    bits = _seeded_bf16(tokens, n, 7 * n + k)
    g = np.random.default_rng(k + n)
    v = (g.standard_normal((n, k)) / np.sqrt(n)).astype(np.float32)
    wt = (g.standard_normal((k, n)) * 0.05).astype(np.float32)
    s = np.where(g.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    res = hooks.rotate_dynamic_asym_int4(to_dev_bf16(bits), group, signs=torch.from_numpy(s).cuda(),
                                         v=torch.from_numpy(v).cuda(), w_t=torch.from_numpy(wt).cuda())
    torch.cuda.synchronize()
    ref = O.quant(O.rotate(O.bf16_to_f32(bits), m, n // m, signs=s, v=v, wt=wt), group)
    _assert_tuple_exact(_tuple_np(res), ref, f"n={n} m={m} k={k}")


def test_large_paley_limits_raise():
    # rows beyond the 32768 channels one workgroup holds (200 x 256), and a
    # per-block rank term on the whole-row Paley path, are not built
    with pytest.raises(ValueError):
        hooks.full_hadamard_rows(torch.zeros((2, 51200), dtype=torch.bfloat16, device="cuda"), None)
    w_t = torch.zeros((4, 9728), dtype=torch.float32, device="cuda")
    v = torch.zeros((9728, 4), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        hooks.rotate_dynamic_asym_int4(torch.zeros((2, 9728), dtype=torch.bfloat16, device="cuda"), 128,
                                       v=v, w_t=w_t, rank_block=128)
