"""GPU parity of the group-asymmetric W4A4 GEMM (narhip_w4a4_gemm).

Against oracle.w4a4_gemm (fp64 sum of the reference-dequantized operands,
pinned to the four-term group form in tests/test_w4a4_cpu.py).  The kernel
sums the exact integer code products per group and combines the terms in
fp32, so every element is required within 2^-18 of sum_i |a_i| |w_i| (the
fp32 rounding of ~n/128 group terms and of the oracle's dequantization).
Cases: ragged token and output counts, the Llama-3.1-8B down_proj reduction
(n = 14336), decode-sized token counts whose reduction is split over
workgroups (partials summed in split order), activations produced by narhip's own rotate-quant path with
weights quantized by the hooks' quantizer.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from narhip import hooks, ops, workloads  # noqa: E402


def operands(rng, t, o, n, b=128):
    a = rng.integers(0, 256, (t, n // 2), dtype=np.uint8)
    w = rng.integers(0, 256, (o, n // 2), dtype=np.uint8)
    f16 = lambda x: np.asarray(x, np.float16).view(np.uint16)  # noqa: E731
    return (a, f16(rng.uniform(0.005, 0.2, (t, n // b))), f16(rng.uniform(-2, 1, (t, n // b))),
            w, f16(rng.uniform(0.001, 0.02, (o, n // b))), f16(rng.uniform(-0.1, 0.05, (o, n // b))))


def run(a, sa, za, w, sw, zw):
    d = lambda x: torch.from_numpy(x).cuda()  # noqa: E731
    h = lambda x: torch.from_numpy(x.view(np.int16)).cuda().view(torch.float16)  # noqa: E731
    y = ops.w4a4_gemm(d(a), h(sa), h(za), d(w), h(sw), h(zw))
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check(y, a, sa, za, w, sw, zw, n):
    ref = O.w4a4_gemm(a, sa, za, w, sw, zw, n)
    da, dw = O.dequant(a, sa, za, n, 128), O.dequant(w, sw, zw, n, 128)
    scale = np.abs(da).astype(np.float64) @ np.abs(dw).astype(np.float64).T
    err = np.abs(y - ref) / scale
    print(f"  max |err| / sum|a||w| = {err.max():.3e}", flush=True)
    assert np.all(np.abs(y - ref) <= 2.0 ** -18 * scale)


@pytest.mark.parametrize("t,o,n", [(1, 128, 128), (37, 200, 1024), (130, 256, 256), (256, 384, 14336),
                                   (64, 1024, 14336), (3, 500, 4096)])
def test_random_operands(t, o, n):
    print(f"[test_random_operands] t={t} o={o} n={n}", flush=True)
    rng = np.random.default_rng(t * 1000 + o)
    ops_ = operands(rng, t, o, n)
    check(run(*ops_), *ops_, n)


@pytest.mark.parametrize("t,o,n", [(130, 256, 14336), (3, 384, 4096), (64, 128, 128)])
def test_code_products_exact(t, o, n):
    """Unit scales and zero offsets: every output is the integer sum of code
    products, exact in fp32 (below 2^24), so the kernel must return it bit for
    bit -- the fp8 reading of the code bytes (0..7 are e4m3 subnormals) and the
    2^18 rescaling lose nothing, with or without the reduction split over
    workgroups (t = 3: decode-sized, split partials)."""
    print(f"[test_code_products_exact] t={t} o={o} n={n}", flush=True)
    rng = np.random.default_rng(t + o + n)
    a = rng.integers(0, 256, (t, n // 2), dtype=np.uint8)
    w = rng.integers(0, 256, (o, n // 2), dtype=np.uint8)
    a[0] = 0x11                                  # all codes 1 (the smallest subnormal) in one row
    w[0] = 0x77                                  # all codes 7 (the largest subnormal)
    ones = lambda r: np.full((r, n // 128), np.float16(1.0)).view(np.uint16)  # noqa: E731
    zero = lambda r: np.zeros((r, n // 128), np.uint16)  # noqa: E731
    y = run(a, ones(t), zero(t), w, ones(o), zero(o))
    qa = O.unpack(a, n).astype(np.int64)
    qw = O.unpack(w, n).astype(np.int64)
    want = qa @ qw.T
    assert want.max() < 2 ** 24
    assert np.array_equal(y, want.astype(np.float32)), np.abs(y - want).max()


def test_extreme_codes_and_zero_scales():
    print("[test_extreme_codes_and_zero_scales]", flush=True)
    rng = np.random.default_rng(3)
    n = 512
    a, sa, za, w, sw, zw = operands(rng, 64, 128, n)
    a[:8] = 0xFF                                  # all codes 15
    w[:, :32] = 0x00                              # a group of zero codes
    sa[9] = np.float16(0).view(np.uint16)         # zero scale row: pure offset
    zw[5] = np.float16(0).view(np.uint16)
    check(run(a, sa, za, w, sw, zw), a, sa, za, w, sw, zw, n)


def test_rotate_quant_activations_times_quantized_weights():
    """A from narhip's E17 block-H128 path, W from the hooks quantizer."""
    print("[test_rotate_quant_activations_times_quantized_weights]", flush=True)
    wl = workloads.e17_3b(tokens=96, k=8)
    x = torch.from_numpy(wl.x.view(np.int16)).cuda().view(torch.bfloat16)
    v, wt = torch.from_numpy(wl.v).cuda(), torch.from_numpy(wl.w_t).cuda()
    codes, scales, zeros = ops.rotate_quant(x, hadamard=(1, 128), v=v, w_t=wt, group=128)
    g = torch.Generator().manual_seed(7)
    weight = (torch.randn((160, wl.n), generator=g) / wl.n ** 0.5).cuda()
    _, ws, wz, wc = hooks.dynamic_asym_int4(weight, 128)
    wpack = ops.pack_codes(wc.reshape(160, wl.n))
    y = ops.w4a4_gemm(codes, scales, zeros, wpack, ws.reshape(160, -1).contiguous(),
                      wz.reshape(160, -1).contiguous())
    torch.cuda.synchronize()
    n16 = lambda t: t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    check(y.cpu().numpy(), codes.cpu().numpy(), n16(scales), n16(zeros), wpack.cpu().numpy(), n16(ws.reshape(160, -1)),
          n16(wz.reshape(160, -1)), wl.n)
