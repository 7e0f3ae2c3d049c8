"""Registration of the torch.ops.narhip operators, checked without a GPU.

Schemas (mutated outputs annotated, everything else read-only), the fake
kernels' output shapes and dtypes under FakeTensorMode on "cuda" tensors (no
device needed), the keyword wrappers traced through them, and that a real CPU
tensor finds no kernel (there is no CPU path).
"""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

from torch._subclasses.fake_tensor import FakeTensorMode  # noqa: E402

from narhip import hooks, ops  # noqa: E402

N = torch.ops.narhip

MUTATING = {
    "rotate_quant_out": {"codes", "scales", "zeros", "rotated"},
    "rank_projection_out": {"partial"},
    "rank_projection_f16_out": {"partial"},
    "group_quant_out": {"codes", "scales", "zeros"},
    "transform_f16_out": {"out"},
    "w4a4_gemm_out": {"out"},
}
FUNCTIONAL = ("rotate_quant", "rank_projection", "group_quant", "transform_f16", "dynamic_asym_int4",
              "hadamard_rows", "dequantize", "w4a4_gemm", "prepare_rank_factors")


@pytest.mark.parametrize("name", list(MUTATING) + list(FUNCTIONAL))
def test_schema_mutations(name):
    schema = getattr(N, name).default._schema
    written = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == MUTATING.get(name, set()), (name, written)
    if name in MUTATING:
        assert len(schema.returns) == 0


def test_fake_shapes():
    with FakeTensorMode():
        dev = "cuda"
        T, n, k = 24, 14336, 32
        x = torch.empty((T, n), dtype=torch.bfloat16, device=dev)
        v = torch.empty((n, k), device=dev)
        wt = torch.empty((k, n), device=dev)
        c, s, z = ops.rotate_quant(x, hadamard=(28, 512), v=v, w_t=wt, group=128)
        assert (c.shape, c.dtype, s.shape, s.dtype, z.shape) == (
            (T, n // 2), torch.uint8, (T, n // 128), torch.float16, (T, n // 128))
        c, s, z = N.group_quant(x, torch.empty((T, 4 * k), device=dev), wt, None, 28, 512, 64, 0)
        assert c.shape == (T, n // 2) and s.shape == (T, n // 64)
        p = N.rank_projection(x, v, None, k, 4, 0)
        assert p.shape == (T, 4 * k) and p.dtype == torch.float32
        xf16 = torch.empty((T, n), dtype=torch.float16, device=dev)
        o = N.transform_f16(xf16, wt, v, None, 128)
        assert o.shape == (T, n) and o.dtype == torch.float16
        deq, sc, zc, codes = hooks.dynamic_asym_int4(torch.empty((2, 3, 256), device=dev), 32)
        assert deq.shape == (2, 3, 256) and deq.dtype == torch.float32
        assert sc.shape == zc.shape == (2, 3, 8) and codes.shape == (2, 3, 8, 32) and codes.dtype == torch.uint8
        h = hooks.full_hadamard_rows(torch.empty((2, 5, 3072), dtype=torch.bfloat16, device=dev), None)
        assert h.shape == (2, 5, 3072) and h.dtype == torch.float32
        d = N.dequantize(c, s, z, n, 64)
        assert d.shape == (T, n) and d.dtype == torch.float32
        y = N.w4a4_gemm(c, s, z, c[:7], s[:7], z[:7], 64)
        assert y.shape == (T, 7) and y.dtype == torch.float32


def test_cpu_tensors_find_no_kernel():
    x = torch.zeros((4, 128), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        N.rotate_quant(x, 1, 128, None, None, None, None, 128, None, 128, 0)
    with pytest.raises(NotImplementedError):
        N.dynamic_asym_int4(torch.zeros((2, 64)), 32)


def test_wrappers_reject_cpu_tensors():
    with pytest.raises(ValueError):
        ops.rotate_quant(torch.zeros((4, 128), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        hooks.dynamic_asym_int4(torch.zeros((2, 64)), 32)
