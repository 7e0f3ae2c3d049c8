"""Launchers fed a factor that reuses a freed factor's device address.

The reference's per-layer loops (nar/e17_v2_fold_verify.py:139-185,
nar/e17_v3.py:206-251) free one layer's Y'/W'' and allocate the next; the
caching allocator returns the same block.  The cached transposes and prepared
MFMA terms must follow the new factor: output equals the oracle for factor B.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest

from helpers import f16_bits, to_dev_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from nar.kernels import r4_fused_v2 as k2  # noqa: E402
from nar.kernels import r4_fused_v3 as k3  # noqa: E402
from narhip import workloads  # noqa: E402
from narhip.factors import cached_transpose  # noqa: E402

REL_ERR = 2.0 ** -21


def layer_factors(n, k, seed):
    rng = np.random.default_rng(seed)
    v = workloads.orthonormal(rng, n, k)
    wt = np.ascontiguousarray(-workloads.orthonormal(rng, n, k).T)
    return v, wt


def rows(tokens, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((tokens, n), generator=g).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def check_layer(out, bits, v, wt):
    n = bits.shape[1]
    rot = O.rotate(O.bf16_to_f32(bits), 1, 128, v=v, wt=wt)
    ref = O.quant(rot, 128)
    rep = O.compare_quant(rot, ref, O.unpack(out.codes.cpu().numpy(), n), f16_bits(out.scales),
                          f16_bits(out.zeros), 128, rel_err=REL_ERR)
    print("  ", rep, flush=True)
    assert rep.within_contract(), rep


@pytest.mark.parametrize("k", [8, 32])
def test_fused_launch_with_reused_factor_address(k):
    n, tokens = 8192, 48
    print(f"[test_fused_launch_with_reused_factor_address] k={k} n={n}", flush=True)
    bits = rows(tokens, n, 77 + k)
    x = to_dev_bf16(bits)
    va, wta = layer_factors(n, k, 1000 + k)
    vb, wtb = layer_factors(n, k, 2000 + k)
    ya = torch.from_numpy(np.ascontiguousarray(va.T)).cuda()
    wa = torch.from_numpy(wta).cuda()
    out = k2.allocate_outputs(tokens, n, x.device)
    k2.launch_nar_fused(x, ya, wa, out)
    torch.cuda.synchronize()
    check_layer(out, bits, va, wta)
    freed = {ya.data_ptr(), wa.data_ptr(), cached_transpose(ya).data_ptr()}
    del ya, wa
    gc.collect()
    yb = torch.empty((k, n), dtype=torch.float32, device="cuda")
    wb = torch.empty((k, n), dtype=torch.float32, device="cuda")
    assert yb.data_ptr() in freed or wb.data_ptr() in freed, "the allocator did not reuse a freed block"
    yb.copy_(torch.from_numpy(np.ascontiguousarray(vb.T)))
    wb.copy_(torch.from_numpy(wtb))
    # the copy bumped the version; recreate fresh tensors at the same address
    # at version 0 as well (a load straight into a new tensor has version 0)
    yb0 = torch.empty(0, device="cuda").set_(yb.untyped_storage(), 0, (k, n))
    wb0 = torch.empty(0, device="cuda").set_(wb.untyped_storage(), 0, (k, n))
    for y_, w_ in ((yb, wb), (yb0, wb0)):
        out = k2.allocate_outputs(tokens, n, x.device)
        k2.launch_nar_fused(x, y_, w_, out)
        torch.cuda.synchronize()
        check_layer(out, bits, vb, wtb)


def test_projection_dot_with_reused_term_address():
    n, k, tokens = 8192, 32, 40
    print("[test_projection_dot_with_reused_term_address]", flush=True)
    bits = rows(tokens, n, 5)
    x = to_dev_bf16(bits)
    kp = k3.padded_rank(k)
    cfg = k3.PROJECTION_CONFIGS[0]
    results = []
    ptr = None
    for seed in (11, 12):
        v, _ = layer_factors(n, k, seed)
        vf = torch.from_numpy(v)
        hi = vf.to(torch.bfloat16)
        mid = (vf - hi.float()).to(torch.bfloat16)
        lo = (vf - hi.float() - mid.float()).to(torch.bfloat16)
        terms = torch.zeros((3, n, kp), dtype=torch.bfloat16)
        terms[0, :, :k], terms[1, :, :k], terms[2, :, :k] = hi, mid, lo
        y_padded = terms.reshape(3 * n, kp).cuda()
        if ptr is not None:
            assert y_padded.data_ptr() == ptr, "the allocator did not reuse the freed block"
        ptr = y_padded.data_ptr()
        partial = torch.empty((tokens, cfg.splits * k), dtype=torch.float32, device="cuda")
        k3.launch_projection_dot(x, y_padded, partial, k, cfg, 3)
        torch.cuda.synchronize()
        u = k2.reduce_partial(partial, k).cpu().numpy()
        u_ref = O.projection(O.bf16_to_f32(bits), v)
        err = np.abs(u - u_ref).max() / np.abs(u_ref).max()
        print(f"   seed {seed}: max rel err {err:.3e}", flush=True)
        assert err <= 1e-5
        results.append(u)
        del y_padded, partial
        gc.collect()
    assert not np.array_equal(results[0], results[1])
