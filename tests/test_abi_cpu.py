"""The C-ABI library loads without a GPU and exports every declared entry point;
host-side validation rejects bad arguments before any device work."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> list[str]:
    text = (ROOT / "include" / "narhip.h").read_text()
    return sorted(set(re.findall(r"\b(narhip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import narhip
    lib = narhip.load()
    names = declared_symbols()
    assert "narhip_rotate_quant" in names and len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name
    assert lib.narhip_abi_version() == 1


@pytest.mark.parametrize("m", [12, 20, 28, 68, 76, 200])
def test_library_paley_equals_oracle(m):
    import narhip
    out = np.zeros((m, m), np.int8)
    assert narhip.load().narhip_paley(m, out.ctypes.data_as(ctypes.c_void_p)) == 0
    assert np.array_equal(out, O.paley(m))


def test_unsupported_paley_order():
    import narhip
    out = np.zeros((24, 24), np.int8)
    lib = narhip.load()
    assert lib.narhip_paley(24, out.ctypes.data_as(ctypes.c_void_p)) == -2
    assert b"24" in lib.narhip_last_error_string()


def _rq(lib, **kw):
    a = dict(x=None, T=4, n=1024, ld=1024, m=1, q=128, signs=None, k=0, nb=1024, v=None, wt=None,
             prepared=None, partial=None, splits=0, group=128, codes=None, scales=None, zeros=None, rot=None,
             dest=None, mode=0, ws=None, wsb=0, stream=None)
    a.update(kw)
    return lib.narhip_rotate_quant(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(n=1000), -1),                       # n % 128
    (dict(q=96), -2),                         # not a power of two
    (dict(q=2048), -2),                       # beyond the built widths
    (dict(m=24, q=128, n=3072), -2),          # no Paley 24
    (dict(m=68, q=256, n=17408), -2),         # Qwen3 order 68: not built
    (dict(q=4096, n=4096, ld=4096, k=8, v=16, wt=16), -2),   # no rank term on the full-row FWHT
    (dict(q=16384, n=16384, ld=16384), -2),   # FWHT rows beyond 8192
    (dict(group=48), -2),
    (dict(k=65, wt=1), -2),
    (dict(m=28, q=512, n=14336, ld=14336, k=32, nb=14336, v=16, wt=16, x=16, codes=16, scales=16, zeros=16), -4),
    (dict(m=28, q=512, n=14336, ld=14336, k=32, nb=14336), -1),   # rank factors missing
    (dict(ld=1000), -1),
    # prepared terms do not stand in for w_t on the paths that read w_t itself
    (dict(k=8, v=16, prepared=16, x=16, codes=16, scales=16, zeros=16), -1),              # k < 16, AUTO
    (dict(m=28, q=512, n=14336, ld=14336, k=32, nb=14336, v=16, prepared=16, x=16, codes=16, scales=16,
          zeros=16, mode=1), -1),                                                          # RANK_EXACT
])
def test_host_validation(kw, code):
    import narhip
    lib = narhip.load()
    assert _rq(lib, **kw) == code
    assert lib.narhip_last_error_string() != b""


def test_workspace_query():
    import narhip
    lib = narhip.load()
    assert lib.narhip_rotate_quant_workspace(8, 1024, 1, 128, 0, 1024, 0, 0, 0, 0) == 0
    exact = lib.narhip_rotate_quant_workspace(8192, 14336, 28, 512, 32, 14336, 0, 0, 0, 1)
    assert exact >= 8192 * 14336 * 4
    mfma = lib.narhip_rotate_quant_workspace(8192, 14336, 28, 512, 32, 14336, 0, 0, 0, 0)
    prepared = lib.narhip_rotate_quant_workspace(8192, 14336, 28, 512, 32, 14336, 0, 0, 1, 0)
    assert mfma - prepared == lib.narhip_rank_factors_bytes(14336, 32) > 0


def test_hadamard_factor_dispatch_order():
    from narhip.ops import hadamard_factors
    assert hadamard_factors(14336) == (28, 512)
    assert hadamard_factors(28672) == (28, 1024)
    assert hadamard_factors(3072) == (12, 256)
    assert hadamard_factors(4096) == (1, 4096)
    with pytest.raises(ValueError):
        hadamard_factors(1000)


def _tf(lib, **kw):
    a = dict(x=None, T=4, n=8192, ld=8192, q=128, v=None, partial=None, splits=0, wt=None, k=0, out=None,
             ws=None, wsb=0, stream=None)
    a.update(kw)
    return lib.narhip_transform_f16(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(q=96), -2),                               # not a power of two
    (dict(q=2048), -2),
    (dict(n=8064, ld=8064, q=256), -2),             # 256 does not divide n
    (dict(k=65, wt=16, v=16), -2),                  # rank beyond the fp16 path
    (dict(ld=8190), -1),
    (dict(k=8, wt=16, partial=16, splits=0), -1),   # partials without splits
    (dict(k=8, wt=16, v=16, x=16, out=16), -4),     # projection workspace missing
    (dict(k=8, x=16, out=16, partial=16, splits=2), -1),   # W^T missing
])
def test_transform_f16_host_validation(kw, code):
    import narhip
    lib = narhip.load()
    assert _tf(lib, **kw) == code
    assert lib.narhip_last_error_string() != b""


def test_transform_f16_workspace_query():
    import narhip
    lib = narhip.load()
    assert lib.narhip_transform_f16_workspace(2048, 14336, 0) == 0
    assert lib.narhip_transform_f16_workspace(2048, 14336, 65) == 0
    # k = 32: fp64 partials in two slices of 16 ranks, plus u
    assert lib.narhip_transform_f16_workspace(2048, 14336, 32) >= 2048 * 32 * (8 + 4)
    ws = lib.narhip_transform_f16_workspace(2048, 14336, 8)
    assert ws >= 2048 * 8 * 4 + 2048 * 8 * 8 and ws % 256 == 0


@pytest.mark.parametrize("k,n,splits,code", [
    (0, 14336, 1, -2), (65, 14336, 1, -2),
    (8, 14336, 3, -1),          # 3 does not divide n
    (8, 14343, 7, -1),          # 7 x 2049: odd channel chunks
])
def test_rank_projection_f16_host_validation(k, n, splits, code):
    import narhip
    lib = narhip.load()
    ld = (n + 7) // 8 * 8
    assert lib.narhip_rank_projection_f16(None, 4, n, ld, None, k, splits, None, None) == code
    assert lib.narhip_last_error_string() != b""


def test_group_quant_requires_w_t_off_the_mfma_path():
    """Kernel B with prepared terms but no w_t: only the MFMA rank path may go on."""
    import narhip
    lib = narhip.load()
    args = [16, 4, 1024, 1024, 1, 128, 16, 1, 8, None, 16, 128, 16, 16, 16, 0, None, 0, None]
    assert lib.narhip_group_quant(*args) == -1
    assert b"w_t" in lib.narhip_last_error_string()
    exact = [16, 4, 14336, 14336, 28, 512, 16, 1, 32, None, 16, 128, 16, 16, 16, 1, None, 0, None]
    assert lib.narhip_group_quant(*exact) == -1


def test_noalloc_host_validation():
    """The allocation-free entry point rejects, before any device work, arguments
    whose scratch exceeds its array (the exact Kronecker path over 2048 rows of
    14336 needs a 117 MB correction buffer) and bad shapes like the other one."""
    import narhip
    lib = narhip.load()
    n = 14336
    assert lib.narhip_rotate_quant_workspace(2048, n, 28, 512, 32, n, 0, 0, 0, 1) > 64 << 20
    rc = lib.narhip_rotate_quant_noalloc(16, 2048, n, n, 28, 512, None, 32, n, 16, 16, None, None, 0, 128,
                                         16, 16, 16, None, None, 1, None)
    assert rc == -4 and b"allocation-free" in lib.narhip_last_error_string()
    rc = lib.narhip_rotate_quant_noalloc(16, 4, 1000, 1000, 1, 128, None, 0, 1000, None, None, None, None, 0,
                                         128, 16, 16, 16, None, None, 0, None)
    assert rc == -1


@pytest.mark.parametrize("rows,n,m,q,code", [
    (0, 9728, 76, 128, 0),          # valid Qwen3 width, nothing to do
    (0, 25600, 200, 128, 0),
    (2, 51200, 200, 256, -2),       # more than one workgroup's 32768 channels
    (2, 9728, 76, 100, -2),         # q not a power of two
    (2, 9728, 68, 128, -2),         # m q != n
    (-1, 9728, 76, 128, -1),
])
def test_large_paley_rows_host_validation(rows, n, m, q, code):
    """The whole-row Paley kernel's host checks (no launch: rows == 0 or an error first)."""
    import narhip
    lib = narhip.load()
    assert lib.narhip_hadamard_rows(None, rows, n, n, m, q, None, None, None) == code


def test_large_paley_tuple_workspace_query():
    import narhip
    lib = narhip.load()
    # x' staged as fp32; with a full-row rank term also u and C (0 = not supported)
    assert lib.narhip_rotate_dynamic_asym_int4_workspace(5, 9728, 76, 128, 0, 9728, 128, 0) >= 4 * 5 * 9728
    assert lib.narhip_rotate_dynamic_asym_int4_workspace(5, 9728, 76, 128, 8, 9728, 128, 0) >= 8 * 5 * 9728
    assert lib.narhip_rotate_dynamic_asym_int4_workspace(5, 9728, 76, 128, 8, 128, 128, 0) == 0   # per block
    assert lib.narhip_rotate_dynamic_asym_int4_workspace(5, 9728, 76, 128, 65, 9728, 128, 0) == 0
