"""GPU parity of the fused rotate -> rank-k -> INT4 op against the CPU oracle.

Exact rank mode: the oracle defines the reference's BLAS products as fp64
sums rounded once, and the exact kernels compute the same sums in fp64, so
codes, scales, zeros and the rotated fp32 rows must be bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits, oracle_for, to_dev_bf16, to_dev_f32
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import ops, workloads  # noqa: E402

SMALL = {
    "kcache_3b": lambda: workloads.kcache_3b(tokens=96),
    "qproj_3b": lambda: workloads.qproj_3b(tokens=24),
    "downproj_8b": lambda: workloads.downproj_8b(tokens=10),
    "vcache_decode_8b": lambda: workloads.vcache_decode_8b(),
    "downproj_70b": lambda: workloads.downproj_70b(tokens=3),
}


def run(w, rank_mode=ops.RANK_EXACT, with_rotated=True):
    x = to_dev_bf16(w.x)
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    rot = torch.empty((w.tokens, w.n), dtype=torch.float32, device="cuda") if with_rotated else None
    dest = None if w.dest_rows is None else torch.from_numpy(w.dest_rows).cuda()
    codes, scales, zeros = ops.rotate_quant(
        x, hadamard=w.hadamard, v=v, w_t=wt, rank_block=w.rank_block, group=w.group,
        rotated=rot, dest_rows=dest, rank_mode=rank_mode, out_rows=w.out_rows)
    torch.cuda.synchronize()
    return codes, scales, zeros, rot


def gathered(w, codes, scales, zeros):
    if w.dest_rows is None:
        return codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros)
    idx = torch.from_numpy(w.dest_rows).cuda()
    return codes[idx].cpu().numpy(), f16_bits(scales[idx]), f16_bits(zeros[idx])


@pytest.mark.parametrize("name", list(SMALL))
def test_small_exact(name):
    print(f"[test_small_exact] {name}", flush=True)
    w = SMALL[name]()
    codes, scales, zeros, rot = run(w)
    ref_rot, ref = oracle_for(w)
    assert np.array_equal(rot.cpu().numpy(), ref_rot), O.rotated_error(rot.cpu().numpy(), ref_rot)
    c, s, z = gathered(w, codes, scales, zeros)
    assert np.array_equal(c, ref.packed)
    assert np.array_equal(s, ref.scales)
    assert np.array_equal(z, ref.zeros)
    deq = O.dequant(c, s, z, w.n, w.group)
    assert np.array_equal(deq, ref.deq)
    x = O.bf16_to_f32(w.x)
    assert f"{O.nmse(ref_rot, deq):.4g}" == f"{O.nmse(ref_rot, ref.deq):.4g}"
    del x


@pytest.mark.parametrize("name", ["kcache_3b", "qproj_3b", "downproj_8b", "vcache_decode_8b"])
def test_full_size_sampled_rows(name):
    """Full-size launch; a seeded sample of rows is checked bit-exactly against the oracle."""
    print(f"[test_full_size_sampled_rows] {name}", flush=True)
    w = workloads.CONFIGS[name]()
    codes, scales, zeros, _ = run(w, with_rotated=False)
    rows = np.sort(np.random.default_rng(7).choice(w.tokens, size=min(12, w.tokens), replace=False))
    rows = np.unique(np.concatenate([rows, [0, w.tokens - 1]]))
    _, ref = oracle_for(w, rows)
    c, s, z = gathered(w, codes, scales, zeros)
    assert np.array_equal(c[rows], ref.packed)
    assert np.array_equal(s[rows], ref.scales)
    assert np.array_equal(z[rows], ref.zeros)
    # size-independent properties over every row: codes in range (nibbles are
    # always 0..15), scales positive and finite, zero <= every dequantized value
    assert np.isfinite(s.view(np.float16).astype(np.float32)).all()
    assert (s.view(np.float16).astype(np.float32) > 0).all()


def test_full_size_70b_sampled_rows():
    print("[test_full_size_70b_sampled_rows]", flush=True)
    w = workloads.downproj_70b()
    codes, scales, zeros, _ = run(w, with_rotated=False)
    rows = np.array([0, 1, 4097, 9999, w.tokens - 1])
    _, ref = oracle_for(w, rows)
    c, s, z = gathered(w, codes, scales, zeros)
    assert np.array_equal(c[rows], ref.packed)
    assert np.array_equal(s[rows], ref.scales)
    assert np.array_equal(z[rows], ref.zeros)


def test_dest_rows_scatter_leaves_other_slots():
    print("[test_dest_rows_scatter_leaves_other_slots]", flush=True)
    w = workloads.vcache_decode_8b()
    x = to_dev_bf16(w.x)
    codes = torch.full((w.out_rows, w.n // 2), 0xA5, dtype=torch.uint8, device="cuda")
    scales = torch.full((w.out_rows, w.n // w.group), -7.0, dtype=torch.float16, device="cuda")
    zeros = torch.full_like(scales, 3.0)
    dest = torch.from_numpy(w.dest_rows).cuda()
    ops.rotate_quant(x, hadamard=w.hadamard, v=to_dev_f32(w.v), w_t=to_dev_f32(w.w_t), rank_block=w.rank_block,
                     group=w.group, codes=codes, scales=scales, zeros=zeros, dest_rows=dest,
                     rank_mode=ops.RANK_EXACT)
    torch.cuda.synchronize()
    mask = torch.ones(w.out_rows, dtype=torch.bool, device="cuda")
    mask[dest] = False
    assert bool((codes[mask] == 0xA5).all())
    assert bool((scales[mask] == -7.0).all()) and bool((zeros[mask] == 3.0).all())
    _, ref = oracle_for(w)
    assert np.array_equal(codes[dest].cpu().numpy(), ref.packed)


def _special_rows(n: int, t: int) -> np.ndarray:
    rng = np.random.default_rng(17)
    base = rng.standard_normal(n).astype(np.float32)
    cases = [np.zeros(n, np.float32), np.full(n, 0.5, np.float32),
             ((np.arange(n) % 15 - 7 + 0.5) / 7).astype(np.float32),
             (64 + base * 0.03125).astype(np.float32), base.copy()]
    cases[-1][0] = 128.0
    rows = np.stack([cases[i % len(cases)] for i in range(t)])
    return O.bf16_bits(rows)


@pytest.mark.parametrize("shape", [(1, 128, 1024, 128), (12, 256, 3072, 64), (28, 512, 14336, 128)])
def test_special_case_suite(shape):
    """zero / constant / rounding_boundary / common_offset / outlier rows
    (quarot-llama3/e28_v2/verify.py:43-49), Hadamard only and with rank-k."""
    m, q, n, b = shape
    print(f"[test_special_case_suite] {shape}", flush=True)
    bits = _special_rows(n, 10)
    x = to_dev_bf16(bits)
    for k in (0, 16):
        rng = np.random.default_rng(k)
        v = workloads.orthonormal(rng, n, k) if k else None
        wt = np.ascontiguousarray(-workloads.orthonormal(rng, n, k).T) if k else None
        rot = torch.empty((10, n), dtype=torch.float32, device="cuda")
        codes, scales, zeros = ops.rotate_quant(x, hadamard=(m, q), v=to_dev_f32(v), w_t=to_dev_f32(wt),
                                                group=b, rotated=rot, rank_mode=ops.RANK_EXACT)
        torch.cuda.synchronize()
        ref_rot = O.rotate(O.bf16_to_f32(bits), m, q, v=v, wt=wt)
        ref = O.quant(ref_rot, b)
        assert np.array_equal(rot.cpu().numpy(), ref_rot)
        assert np.array_equal(codes.cpu().numpy(), ref.packed)
        assert np.array_equal(f16_bits(scales), ref.scales)
        assert np.array_equal(f16_bits(zeros), ref.zeros)


@pytest.mark.parametrize("tokens", [0, 1, 3, 17])
def test_ragged_tokens_strided_rows_and_signs(tokens):
    print(f"[test_ragged_tokens_strided_rows_and_signs] {tokens}", flush=True)
    n, ld = 3072, 3072 + 64
    rng = np.random.default_rng(tokens)
    full = O.bf16_bits(rng.standard_normal((max(tokens, 1), ld)).astype(np.float32) * 3)
    signs = rng.choice(np.array([-1.0, 1.0], np.float32), size=n)
    xd = to_dev_bf16(full)[:tokens, :n]
    for (m, q) in ((12, 256), (1, 128), (1, 512)):
        codes, scales, zeros = ops.rotate_quant(xd, hadamard=(m, q), signs=to_dev_f32(signs), group=64,
                                                rank_mode=ops.RANK_EXACT)
        torch.cuda.synchronize()
        if tokens == 0:
            assert codes.shape == (0, n // 2)
            continue
        ref = O.quant(O.rotate(O.bf16_to_f32(full[:tokens, :n]), m, q, signs=signs), 64)
        assert np.array_equal(codes.cpu().numpy(), ref.packed)
        assert np.array_equal(f16_bits(scales), ref.scales)
        assert np.array_equal(f16_bits(zeros), ref.zeros)


def test_dequantize_kernel():
    print("[test_dequantize_kernel]", flush=True)
    w = SMALL["qproj_3b"]()
    codes, scales, zeros, _ = run(w, with_rotated=False)
    deq = ops.dequantize(codes, scales, zeros, w.n, w.group).cpu().numpy()
    ref = O.dequant(codes.cpu().numpy(), f16_bits(scales), f16_bits(zeros), w.n, w.group)
    assert np.array_equal(deq, ref)


def test_invalid_arguments_raise_value_error():
    x = torch.zeros((4, 1000), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.rotate_quant(x, hadamard=(1, 128))            # 1000 % 128
    x = torch.zeros((4, 1024), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.rotate_quant(x, hadamard=(1, 128), group=48)
    with pytest.raises(ValueError):
        ops.rotate_quant(x.float(), hadamard=(1, 128))
