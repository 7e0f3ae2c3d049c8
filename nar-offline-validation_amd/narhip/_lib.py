"""ctypes binding of libnarhip.so (include/narhip.h).

The library is built in-tree by narhip/build.py.  Loading fails loudly when it
is missing: there is no CPU or PyTorch fallback for any operator.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnarhip.so"

NARHIP_OK = 0
NARHIP_EINVAL = -1
NARHIP_EUNSUPPORTED = -2
NARHIP_EHIP = -3
NARHIP_EWORKSPACE = -4

RANK_AUTO = 0
RANK_EXACT = 1
RANK_MFMA = 2

EXPORTS = (
    "narhip_abi_version", "narhip_last_error_string", "narhip_paley",
    "narhip_rotate_quant", "narhip_rotate_quant_workspace", "narhip_rotate_quant_noalloc",
    "narhip_rank_factors_bytes", "narhip_prepare_rank_factors",
    "narhip_rank_projection", "narhip_group_quant", "narhip_dequantize",
    "narhip_dynamic_asym_int4", "narhip_rotate_dynamic_asym_int4", "narhip_rotate_dynamic_asym_int4_workspace",
    "narhip_hadamard_rows", "narhip_transform_f16",
    "narhip_transform_f16_workspace", "narhip_rank_projection_f16", "narhip_w4a4_gemm", "narhip_w4a4_workspace",
    "narhip_mfma_probe",
)

_lib: ctypes.CDLL | None = None

c_i32, c_i64, c_sz, c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run narhip/build.py (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.narhip_abi_version.restype = ctypes.c_int
    lib.narhip_last_error_string.restype = ctypes.c_char_p
    lib.narhip_paley.argtypes = [c_i32, c_p]
    lib.narhip_rotate_quant.argtypes = [
        c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p,
        c_i32, c_i64, c_p, c_p, c_p, c_p, c_i32,
        c_i32, c_p, c_p, c_p, c_p, c_p, c_i32, c_p, c_sz, c_p]
    lib.narhip_rotate_quant_noalloc.argtypes = lib.narhip_rotate_quant.argtypes[:-3] + [c_p]
    lib.narhip_rotate_quant_workspace.argtypes = [c_i64, c_i64, c_i32, c_i32, c_i32, c_i64, c_i32, c_i32,
                                                  c_i32, c_i32]
    lib.narhip_rotate_quant_workspace.restype = c_sz
    lib.narhip_rank_factors_bytes.argtypes = [c_i64, c_i32]
    lib.narhip_rank_factors_bytes.restype = c_sz
    lib.narhip_prepare_rank_factors.argtypes = [c_p, c_p, c_i64, c_i32, c_p, c_sz, c_p]
    lib.narhip_rank_projection.argtypes = [c_p, c_i64, c_i64, c_i64, c_p, c_p, c_i32, c_i32, c_p, c_i32, c_p]
    lib.narhip_group_quant.argtypes = [
        c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_i32, c_i32, c_p, c_p, c_i32,
        c_p, c_p, c_p, c_i32, c_p, c_sz, c_p]
    lib.narhip_dequantize.argtypes = [c_p, c_p, c_p, c_i64, c_i64, c_i32, c_p, c_p]
    lib.narhip_dynamic_asym_int4.argtypes = [c_p, c_i32, c_i64, c_i64, c_i32, c_p, c_p, c_p, c_p, c_p]
    lib.narhip_rotate_dynamic_asym_int4.argtypes = [c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_i32, c_i64,
                                                    c_p, c_p, c_i32, c_p, c_p, c_p, c_p, c_i32, c_p, c_sz, c_p]
    lib.narhip_rotate_dynamic_asym_int4_workspace.argtypes = [c_i64, c_i64, c_i32, c_i32, c_i32, c_i64, c_i32,
                                                              c_i32]
    lib.narhip_rotate_dynamic_asym_int4_workspace.restype = c_sz
    lib.narhip_hadamard_rows.argtypes = [c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_p, c_p]
    lib.narhip_transform_f16.argtypes = [c_p, c_i64, c_i64, c_i64, c_i32, c_p, c_p, c_i32, c_p, c_i32, c_p, c_p,
                                         c_sz, c_p]
    lib.narhip_transform_f16_workspace.argtypes = [c_i64, c_i64, c_i32]
    lib.narhip_transform_f16_workspace.restype = c_sz
    lib.narhip_rank_projection_f16.argtypes = [c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_i32, c_p, c_p]
    lib.narhip_w4a4_gemm.argtypes = [c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_p, c_i64, c_p,
                                     c_sz, c_p]
    lib.narhip_w4a4_workspace.argtypes = [c_i64, c_i64, c_i64]
    lib.narhip_w4a4_workspace.restype = c_sz
    lib.narhip_mfma_probe.argtypes = [c_p, c_p, c_p, c_p]
    for name in ("narhip_paley", "narhip_rotate_quant", "narhip_rotate_quant_noalloc", "narhip_rank_projection",
                 "narhip_prepare_rank_factors",
                 "narhip_group_quant", "narhip_dequantize", "narhip_dynamic_asym_int4",
                 "narhip_rotate_dynamic_asym_int4", "narhip_hadamard_rows",
                 "narhip_transform_f16", "narhip_rank_projection_f16", "narhip_w4a4_gemm", "narhip_mfma_probe"):
        getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Map a negative return code to the reference's exception types."""
    if rc == NARHIP_OK:
        return
    msg = load().narhip_last_error_string().decode(errors="replace")
    if rc in (NARHIP_EINVAL, NARHIP_EUNSUPPORTED, NARHIP_EWORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)
