"""The W4A4 consumer's oracle and host checks (no GPU).

oracle.w4a4_gemm (each operand dequantized as the reference's dequantize, the
products summed in fp64) is pinned against the per-group four-term form of
quarot-llama3/e28_v2/docs/quantizer_contract.md:134-140 evaluated exactly in
integers and fp64, and against a brute-force fp64 sum on a tiny case; a
formula with one term dropped fails.  The C-ABI rejects bad arguments before
any device work.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O


def operands(rng, t, o, n, b=128):
    a = rng.integers(0, 256, (t, n // 2), dtype=np.uint8)
    w = rng.integers(0, 256, (o, n // 2), dtype=np.uint8)
    f16 = lambda x: np.asarray(x, np.float16).view(np.uint16)  # noqa: E731
    return (a, f16(rng.uniform(0.005, 0.2, (t, n // b))), f16(rng.uniform(-2, 1, (t, n // b))),
            w, f16(rng.uniform(0.001, 0.02, (o, n // b))), f16(rng.uniform(-0.1, 0.05, (o, n // b))))


def test_group_formula_pins_the_oracle():
    rng = np.random.default_rng(1)
    n = 384
    a, sa, za, w, sw, zw = operands(rng, 5, 7, n)
    exact = O.w4a4_group_formula(a, sa, za, w, sw, zw, n)
    # brute force in fp64 with unrounded dequantization
    qa, qw = O.unpack(a, n).astype(np.float64), O.unpack(w, n).astype(np.float64)
    da = qa * np.repeat(O.f16_bits_to_f32(sa), 128, 1) + np.repeat(O.f16_bits_to_f32(za), 128, 1)
    dw = qw * np.repeat(O.f16_bits_to_f32(sw), 128, 1) + np.repeat(O.f16_bits_to_f32(zw), 128, 1)
    brute = np.array([[sum(da[i, j] * dw[k, j] for j in range(n)) for k in range(7)] for i in range(5)])
    np.testing.assert_allclose(exact, brute, rtol=1e-12, atol=1e-12)
    scale = np.abs(da) @ np.abs(dw).T
    got = O.w4a4_gemm(a, sa, za, w, sw, zw, n)
    assert np.all(np.abs(got - exact) <= 2.0 ** -21 * scale)
    # planted mistake: the zA zW |g| term dropped
    wrong = exact - 128 * np.einsum("tg,og->to", O.f16_bits_to_f32(za).astype(np.float64),
                                    O.f16_bits_to_f32(zw).astype(np.float64))
    assert np.abs(wrong - brute).max() > 1e-3 * np.abs(brute).max()


def _call(lib, **kw):
    a = dict(ac=16, as_=16, az=16, T=4, wc=16, ws=16, wz=16, O=8, n=256, group=128, out=16, ldo=8, wsp=None,
             wsb=0, stream=None)
    a.update(kw)
    return lib.narhip_w4a4_gemm(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(group=64), -2),
    (dict(n=200), -1),
    (dict(ldo=4), -1),
    (dict(out=None), -1),
    (dict(ac=8), -1),          # codes not 16-byte aligned
    (dict(T=-1), -1),
    (dict(T=64, O=4096, n=14336, ldo=4096), -4),    # split reduction needs its workspace
])
def test_w4a4_host_validation(kw, code):
    import narhip
    lib = narhip.load()
    assert _call(lib, **kw) == code
    assert lib.narhip_last_error_string() != b""


def test_w4a4_empty_is_ok():
    import narhip
    assert _call(narhip.load(), T=0) == 0


def test_w4a4_workspace_query():
    import narhip
    lib = narhip.load()
    assert lib.narhip_w4a4_workspace(8192, 4096, 14336) == 0          # 2048 output tiles: no split
    ws = lib.narhip_w4a4_workspace(64, 4096, 14336)
    assert ws > 0 and ws % (4 * 64 * 4096) == 0
