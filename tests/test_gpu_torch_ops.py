"""The torch.ops.narhip operators: dispatcher registration, fake kernels, compile.

``torch.library.opcheck`` runs every registered operator on real GPU inputs
and checks its schema (declared mutations are the only mutations), its fake
kernel (output shapes, dtypes and strides equal the real ones) and its trace
through AOT dispatch with dynamic shapes (same results as eager).  Then the
drop-in wrappers are compiled with ``torch.compile(backend="aot_eager",
fullgraph=True)`` (a graph break fails the compile) and must return the eager
call's bits.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import to_dev_bf16, to_dev_f32

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from narhip import hooks, ops, workloads  # noqa: E402

N = torch.ops.narhip


def _dev(w):
    x = to_dev_bf16(w.x)
    return x, to_dev_f32(w.v), to_dev_f32(w.w_t)


def _check(op, args, label):
    print(f"[opcheck] {label}", flush=True)
    torch.library.opcheck(op, args)


def _quant_buffers(rows, n, group, device="cuda"):
    return (torch.zeros((rows, n // 2), dtype=torch.uint8, device=device),
            torch.zeros((rows, n // group), dtype=torch.float16, device=device),
            torch.zeros((rows, n // group), dtype=torch.float16, device=device))


def test_opcheck_rotate_quant():
    w = workloads.downproj_8b(32)
    x, v, wt = _dev(w)
    prep = N.prepare_rank_factors(v, wt, w.n, w.k)
    _check(N.prepare_rank_factors, (v, wt, w.n, w.k), "prepare_rank_factors")
    _check(N.rotate_quant, (x, 28, 512, None, v, wt, prep, w.n, None, 128, ops.RANK_AUTO),
           "rotate_quant downproj_8b[32] auto")
    q = workloads.qproj_3b(48)
    xq, vq, wq = _dev(q)
    _check(N.rotate_quant, (xq, 12, 256, None, vq, wq, None, q.n, None, 64, ops.RANK_EXACT),
           "rotate_quant qproj_3b[48] exact")
    kc = workloads.kcache_3b(40)
    xk, vk, wk = _dev(kc)
    signs = torch.where(torch.arange(kc.n, device="cuda") % 3 == 0, -1.0, 1.0).float()
    _check(N.rotate_quant, (xk, 1, 128, signs, vk, wk, None, 128, None, 32, ops.RANK_AUTO),
           "rotate_quant kcache_3b[40] per-head rank, signs")


def test_opcheck_rotate_quant_out_scatter():
    w = workloads.vcache_decode_8b(batch=8, slots=4)
    x, v, wt = _dev(w)
    dest = torch.from_numpy(w.dest_rows).cuda()
    codes, scales, zeros = _quant_buffers(w.out_rows, w.n, w.group)
    rot = torch.zeros((w.tokens, w.n), dtype=torch.float32, device="cuda")
    _check(N.rotate_quant_out, (x, 1, 128, None, v, wt, None, 128, None, 32, dest, ops.RANK_AUTO,
                                codes, scales, zeros, rot), "rotate_quant_out vcache scatter + rotated")


def test_opcheck_kernel_a_and_b():
    w = workloads.e17_8b(tokens=24, k=8)
    x, v, wt = _dev(w)
    splits = 4
    partial = torch.zeros((w.tokens, splits * w.k), dtype=torch.float32, device="cuda")
    _check(N.rank_projection_out, (x, v, None, w.k, ops.RANK_EXACT, partial), "rank_projection_out exact")
    _check(N.rank_projection, (x, v, None, w.k, splits, ops.RANK_EXACT), "rank_projection exact")
    w32 = workloads.e17_8b(tokens=24, k=32)
    x32, v32, wt32 = _dev(w32)
    prep = N.prepare_rank_factors(v32, wt32, w32.n, 32)
    _check(N.rank_projection, (x32, None, prep, 32, 1, ops.RANK_MFMA), "rank_projection mfma")
    N.rank_projection_out(x, v, None, w.k, ops.RANK_EXACT, partial)
    codes, scales, zeros = _quant_buffers(w.tokens, w.n, 128)
    _check(N.group_quant_out, (x, partial, wt, None, 1, 128, 128, ops.RANK_AUTO, codes, scales, zeros),
           "group_quant_out")
    _check(N.group_quant, (x, partial, wt, None, 1, 128, 128, ops.RANK_AUTO), "group_quant")


def test_opcheck_transform_f16():
    w = workloads.e28("8b", tokens=20)
    x = torch.from_numpy(w.x.view(np.float16)).cuda()
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    partial = torch.zeros((w.tokens, 2 * w.k), dtype=torch.float32, device="cuda")
    _check(N.rank_projection_f16_out, (x, v, partial), "rank_projection_f16_out")
    N.rank_projection_f16_out(x, v, partial)
    out = torch.zeros((w.tokens, w.n), dtype=torch.float16, device="cuda")
    _check(N.transform_f16_out, (x, wt, None, partial, 128, out), "transform_f16_out from partials")
    _check(N.transform_f16, (x, wt, v, None, 128), "transform_f16 from v")


def test_opcheck_hooks_dequantize_w4a4():
    g = torch.Generator(device="cuda").manual_seed(3)
    xf = torch.randn((2, 3, 256), device="cuda", generator=g)
    _check(N.dynamic_asym_int4, (xf, 32), "dynamic_asym_int4 fp32")
    _check(N.dynamic_asym_int4, (xf.to(torch.bfloat16), 128), "dynamic_asym_int4 bf16")
    xb = torch.randn((6, 3072), device="cuda", generator=g).to(torch.bfloat16)
    signs = torch.where(torch.arange(3072, device="cuda") % 5 == 0, -1.0, 1.0).float()
    _check(N.hadamard_rows, (xb, 12, 256, signs), "hadamard_rows 12 x 256")
    xq = torch.randn((3, 9728), device="cuda", generator=g).to(torch.bfloat16)
    _check(N.hadamard_rows, (xq, 76, 128, None), "hadamard_rows 76 x 128 (Paley rows)")
    vq = torch.randn((9728, 8), device="cuda", generator=g) / 100.0
    wq = torch.randn((8, 9728), device="cuda", generator=g) / 20.0
    _check(N.rotate_dynamic_asym_int4, (xq, 76, 128, None, vq, wq, 9728, 128, ops.RANK_AUTO),
           "rotate_dynamic_asym_int4 76 x 128, full-row rank 8")
    a = torch.randn((16, 512), device="cuda", generator=g).to(torch.bfloat16)
    wgt = torch.randn((24, 512), device="cuda", generator=g).to(torch.bfloat16)
    ca, sa, za = N.rotate_quant(a, 1, 128, None, None, None, None, 512, None, 128, ops.RANK_AUTO)
    cw, sw, zw = N.rotate_quant(wgt, 1, 128, None, None, None, None, 512, None, 128, ops.RANK_AUTO)
    _check(N.dequantize, (ca, sa, za, 512, 128), "dequantize")
    _check(N.w4a4_gemm, (ca, sa, za, cw, sw, zw, 128), "w4a4_gemm")
    out = torch.zeros((16, 24), dtype=torch.float32, device="cuda")
    _check(N.w4a4_gemm_out, (ca, sa, za, cw, sw, zw, 128, out), "w4a4_gemm_out")


def _same(a, b):
    for u, v in zip(a, b):
        assert u.shape == v.shape and u.dtype == v.dtype
        assert torch.equal(u.view(torch.uint8) if u.dtype != torch.uint8 else u,
                           v.view(torch.uint8) if v.dtype != torch.uint8 else v)


def test_compile_rotate_quant_fullgraph():
    torch._dynamo.reset()
    w = workloads.downproj_8b(48)
    x, v, wt = _dev(w)
    prep = ops.prepare_rank_factors(v, wt, w.n, w.k)

    def fused(x, v, wt, prep):
        return ops.rotate_quant(x, hadamard=(28, 512), v=v, w_t=wt, prepared=prep, group=128)

    eager = fused(x, v, wt, prep)
    compiled = torch.compile(fused, backend="aot_eager", fullgraph=True)
    print("[compile] rotate_quant downproj_8b[48]", flush=True)
    _same(compiled(x, v, wt, prep), eager)
    # a second token count through the same compiled function
    w2 = workloads.downproj_8b(80)
    x2 = to_dev_bf16(w2.x)
    _same(compiled(x2, v, wt, prep), fused(x2, v, wt, prep))


def test_compile_out_variants_fullgraph():
    torch._dynamo.reset()
    w = workloads.vcache_decode_8b(batch=8, slots=4)
    x, v, wt = _dev(w)
    dest = torch.from_numpy(w.dest_rows).cuda()

    def scatter(x, v, wt, dest, codes, scales, zeros):
        ops.rotate_quant(x, hadamard=(1, 128), v=v, w_t=wt, rank_block=128, group=32, codes=codes,
                         scales=scales, zeros=zeros, dest_rows=dest)
        return hooks.dynamic_asym_int4(ops.dequantize(codes, scales, zeros, w.n, 32), 32)

    bufs_e = _quant_buffers(w.out_rows, w.n, 32)
    bufs_c = _quant_buffers(w.out_rows, w.n, 32)
    eager = scatter(x, v, wt, dest, *bufs_e)
    compiled = torch.compile(scatter, backend="aot_eager", fullgraph=True)
    print("[compile] rotate_quant_out scatter + dequantize + dynamic_asym_int4", flush=True)
    got = compiled(x, v, wt, dest, *bufs_c)
    _same(bufs_c, bufs_e)
    _same(got, eager)


def test_cpu_tensor_finds_no_kernel():
    x = torch.zeros((4, 128), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        N.rotate_quant(x, 1, 128, None, None, None, None, 128, None, 128, ops.RANK_AUTO)
