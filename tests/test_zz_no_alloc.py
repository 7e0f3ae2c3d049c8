"""narhip_rotate_quant_noalloc against narhip_rotate_quant, through the C ABI.

The allocation-free entry point takes its scratch from the library's per-device
array instead of a workspace argument.  For each path that uses scratch (the
MFMA rank path, chunked to fit the array when the tokens need more; the exact
Kronecker path; the block-H_128 fp64 projection path) and for paths that use
none, two calls in a row -- the second with fewer tokens, so it runs over
scratch the first call left behind -- must give the allocating entry point's
codes, scales, zeros and rotated rows bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest

from helpers import to_dev_bf16, to_dev_f32

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from narhip import _lib, ops, workloads  # noqa: E402

SCRATCH = 64 << 20


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _call(noalloc, x, w, v, wt, prepared, mode, dest=None, rows=None):
    T, n = x.shape
    m, q = w.hadamard
    k = 0 if wt is None else int(wt.shape[0])
    nb = n if w.rank_block is None else w.rank_block
    rows = T if rows is None else rows
    codes = torch.full((rows, n // 2), 0xAA, dtype=torch.uint8, device="cuda")
    scales = torch.full((rows, n // w.group), 7.0, dtype=torch.float16, device="cuda")
    zeros = torch.full((rows, n // w.group), 7.0, dtype=torch.float16, device="cuda")
    rot = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    head = (_p(x), T, n, x.stride(0), m, q, None, k, nb, _p(v), _p(wt), _p(prepared), None, 0, w.group,
            _p(codes), _p(scales), _p(zeros), _p(rot), _p(dest), mode)
    if noalloc:
        rc = lib.narhip_rotate_quant_noalloc(*head, stream)
    else:
        ws_bytes = lib.narhip_rotate_quant_workspace(T, n, m, q, k, nb, 0, 0, int(prepared is not None), mode)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if ws_bytes else None
        rc = lib.narhip_rotate_quant(*head, _p(ws), ws_bytes, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return codes, scales, zeros, rot


def _equal(a, b, what):
    for name, u, v in zip(("codes", "scales", "zeros", "rotated"), a, b):
        assert torch.equal(u.view(torch.uint8), v.view(torch.uint8)), f"{what}: {name} differ"


CASES = {
    # name: (workload factory(tokens), first tokens, second tokens, rank mode, prepared)
    "downproj_8b_mfma_chunked": (workloads.downproj_8b, 1200, 300, ops.RANK_AUTO, False),
    "downproj_8b_mfma_prepared": (workloads.downproj_8b, 1500, 257, ops.RANK_AUTO, True),
    "qproj_3b_mfma": (workloads.qproj_3b, 700, 96, ops.RANK_AUTO, False),
    "downproj_8b_exact": (workloads.downproj_8b, 96, 40, ops.RANK_EXACT, False),
    "e17_8b_k8_fp64_projection": (lambda t: workloads.e17_8b(tokens=t, k=8), 512, 100, ops.RANK_AUTO, False),
    "kcache_3b_per_head": (workloads.kcache_3b, 512, 64, ops.RANK_AUTO, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_matches_workspace_entry_point(name):
    make, t1, t2, mode, use_prep = CASES[name]
    w = make(t1)
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    prep = ops.prepare_rank_factors(v, wt, w.n, w.k) if use_prep else None
    lib = _lib.load()
    need = lib.narhip_rotate_quant_workspace(t1, w.n, *w.hadamard, w.k, w.rank_block or w.n, 0, 0,
                                             int(use_prep), mode)
    print(f"[noalloc] {name}: T={t1} then {t2}, n={w.n}, k={w.k}, workspace of the allocating call "
          f"{need / 2**20:.1f} MiB", flush=True)
    for t in (t1, t2):
        x = to_dev_bf16(w.x[:t])
        ref = _call(False, x, w, v, wt, prep, mode)
        got = _call(True, x, w, v, wt, prep, mode)
        _equal(got, ref, f"{name} T={t}")


def test_noalloc_scatter_decode():
    w = workloads.vcache_decode_8b(batch=64, slots=64)
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    dest = torch.from_numpy(w.dest_rows).cuda()
    for b in (64, 24):
        print(f"[noalloc] vcache_decode_8b scatter batch {b}", flush=True)
        x = to_dev_bf16(w.x[:b])
        ref = _call(False, x, w, v, wt, None, ops.RANK_AUTO, dest=dest[:b], rows=w.out_rows)
        got = _call(True, x, w, v, wt, None, ops.RANK_AUTO, dest=dest[:b], rows=w.out_rows)
        _equal(got, ref, f"vcache scatter batch {b}")


def test_noalloc_rejects_beyond_its_scratch():
    w = workloads.downproj_8b(8)
    lib = _lib.load()
    assert lib.narhip_rotate_quant_workspace(2048, w.n, 28, 512, 32, w.n, 0, 0, 0, ops.RANK_EXACT) > SCRATCH
    x = torch.zeros((2048, w.n), dtype=torch.bfloat16, device="cuda")
    v, wt = to_dev_f32(w.v), to_dev_f32(w.w_t)
    codes = torch.empty((2048, w.n // 2), dtype=torch.uint8, device="cuda")
    sz = torch.empty((2048, w.n // 128), dtype=torch.float16, device="cuda")
    rc = lib.narhip_rotate_quant_noalloc(_p(x), 2048, w.n, w.n, 28, 512, None, 32, w.n, _p(v), _p(wt), None,
                                         None, 0, 128, _p(codes), _p(sz), _p(sz), None, None, ops.RANK_EXACT,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.NARHIP_EWORKSPACE
    assert b"allocation-free" in lib.narhip_last_error_string()
