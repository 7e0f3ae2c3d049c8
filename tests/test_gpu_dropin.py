"""The drop-in launcher modules on the GPU against the oracle.

Call sites written for the reference (nar/kernels/r4_fused_v2.py,
nar/kernels/r4_fused_v3.py) run unchanged and produce the oracle's INT4 output:
bit-exact on the exact paths (k = 0, k = 8), within the tie contract on the
MFMA path (k = 32).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f16_bits, to_dev_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from nar.kernels import r4_fused_v2 as k2  # noqa: E402
from nar.kernels import r4_fused_v3 as k3  # noqa: E402
from narhip import workloads  # noqa: E402

REL_ERR = 2.0 ** -21


def factors(n, k, seed):
    rng = np.random.default_rng(seed)
    v = workloads.orthonormal(rng, n, k)
    wt = np.ascontiguousarray(-workloads.orthonormal(rng, n, k).T)
    return v, wt


def e17_rows(tokens, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((tokens, n), generator=g, dtype=torch.float32).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def oracle_pack(bits, v, wt, m=1, q=128, group=128):
    rot = O.rotate(O.bf16_to_f32(bits), m, q, v=v, wt=wt)
    return rot, O.quant(rot, group)


def check(out, bits, v, wt, exact, m=1, q=128, group=128):
    n = bits.shape[1]
    rot, ref = oracle_pack(bits, v, wt, m, q, group)
    codes, s, z = out.codes.cpu().numpy(), f16_bits(out.scales), f16_bits(out.zeros)
    if exact:
        assert np.array_equal(codes, ref.packed)
        assert np.array_equal(s, ref.scales) and np.array_equal(z, ref.zeros)
    else:
        rep = O.compare_quant(rot, ref, O.unpack(codes, n), s, z, group, rel_err=REL_ERR)
        print("  ", rep)
        assert rep.within_contract(), rep


@pytest.mark.parametrize("k,n", [(8, 8192), (32, 14336)])
def test_v2_launch_nar(k, n):
    print(f"[test_v2_launch_nar] k={k} n={n}", flush=True)
    tokens = 40
    bits = e17_rows(tokens, n, 20260902 + n + k)
    v, wt = factors(n, k, k)
    x = to_dev_bf16(bits)
    y_t = torch.from_numpy(np.ascontiguousarray(v.T)).cuda()
    w = torch.from_numpy(wt).cuda()
    splits = k2.split_count(tokens, n)
    partial = k2.allocate_partial(tokens, k, splits, x.device)
    outputs = k2.allocate_outputs(tokens, n, x.device)
    u = k2.launch_nar(x, y_t, w, outputs, partial)
    torch.cuda.synchronize()
    u_ref = O.projection(O.bf16_to_f32(bits), v)
    u_red = k2.reduce_partial(u, k).cpu().numpy()
    assert np.abs(u_red - u_ref).max() <= 1e-5 * np.abs(u_ref).max()
    # split partials are rounded to fp32 per split, so even the fp64 path can
    # move u by an ulp: the tie contract applies to both ranks
    check(outputs, bits, v, wt, exact=False)
    deq = k2.dequantize(outputs, n).cpu().numpy()
    assert np.array_equal(deq, O.dequant(outputs.codes.cpu().numpy(), f16_bits(outputs.scales),
                                         f16_bits(outputs.zeros), n, 128))


def test_v2_fused_hadamard_and_kronecker_extension():
    print("[test_v2_fused_hadamard_and_kronecker_extension]", flush=True)
    tokens, n, k = 24, 14336, 32
    bits = e17_rows(tokens, n, 5)
    v, wt = factors(n, k, 3)
    x = to_dev_bf16(bits)
    y_t = torch.from_numpy(np.ascontiguousarray(v.T)).cuda()
    w = torch.from_numpy(wt).cuda()
    out = k2.allocate_outputs(tokens, n, x.device)
    k2.launch_nar_fused(x, y_t, w, out)
    torch.cuda.synchronize()
    check(out, bits, v, wt, exact=False)
    had = k2.allocate_outputs(tokens, n, x.device)
    k2.launch_hadamard(x, had)
    torch.cuda.synchronize()
    check(had, bits, None, None, exact=True)
    kron = k2.allocate_outputs(tokens, n, x.device)
    k2.launch_nar_fused(x, y_t, w, kron, hadamard=(28, 512))
    torch.cuda.synchronize()
    check(kron, bits, v, wt, exact=False, m=28, q=512)


def test_v3_projection_dot_and_launch_nar():
    print("[test_v3_projection_dot_and_launch_nar]", flush=True)
    tokens, n, k = 48, 8192, 32
    bits = e17_rows(tokens, n, 11)
    v, wt = factors(n, k, 9)
    x = to_dev_bf16(bits)
    y = torch.from_numpy(v)
    hi = y.to(torch.bfloat16)
    lo = (y - hi.float()).to(torch.bfloat16)
    third = (y - hi.float() - lo.float()).to(torch.bfloat16)
    kp = k3.padded_rank(k)
    terms = torch.zeros((3, n, kp), dtype=torch.bfloat16)
    terms[0, :, :k], terms[1, :, :k], terms[2, :, :k] = hi, lo, third
    y_padded = terms.reshape(3 * n, kp).contiguous().cuda()
    w = torch.from_numpy(wt).cuda()
    for cfg in (k3.PROJECTION_CONFIGS[0], k3.PROJECTION_CONFIGS[2]):
        partial = k3.allocate_partial(tokens, k, cfg.splits, x.device)
        k3.launch_projection_dot(x, y_padded, partial, k, cfg, 3)
        out = k3.allocate_outputs(tokens, n, x.device)
        k3.launch_nar(x, w, out, partial, k, k3.TILE_CONFIGS[4])
        torch.cuda.synchronize()
        check(out, bits, v, wt, exact=False)
    had = k3.allocate_outputs(tokens, n, x.device)
    k3.launch_hadamard(x, had, k3.TILE_CONFIGS[0])
    torch.cuda.synchronize()
    check(had, bits, None, None, exact=True)


def test_v2_error_behaviour():
    x = torch.zeros((8, 256), dtype=torch.bfloat16, device="cuda")
    out = k2.allocate_outputs(8, 256, x.device)
    partial = k2.allocate_partial(8, 16, 1, x.device)
    w = torch.zeros((16, 256), device="cuda")
    with pytest.raises(ValueError):
        k2.launch_nar(x, w, w, out, partial)                      # k=16 not in (8, 32)
    xt = torch.zeros((256, 8), dtype=torch.bfloat16, device="cuda").t()
    with pytest.raises(ValueError):
        k2.launch_hadamard(xt, out)                               # non-contiguous
