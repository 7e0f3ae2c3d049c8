"""The narhip operators, registered with the torch dispatcher (namespace ``narhip``).

Each operator is a ``torch.library.custom_op`` over one entry point of
libnarhip.so, with a fake (meta) implementation, so the calls are visible to
the dispatcher, to functionalization and to ``torch.compile`` (no graph break)
and run on the current stream of their tensors' device.  The ``*_out`` forms
write into caller-allocated outputs (the reference's launchers take their
outputs preallocated, nar/kernels/r4_fused_v2.py:306-350,
quarot-llama3/nar_r4_kernel.py:256-275) and declare them in ``mutates_args``;
the other forms allocate and return their outputs.

The keyword-friendly wrappers with the reference's argument checks are in
``narhip.ops`` and ``narhip.hooks``; they call these operators.  Workspaces
are allocated inside the operator from torch's caching allocator.  Only device
kernels are registered (``device_types="cuda"``, which is HIP on ROCm): a CPU
tensor finds no kernel and raises.

Operator dispatch costs about 25-35 us of host time per call on top of the C
call; callers on a latency budget of a few microseconds bind the C ABI
(include/narhip.h) directly.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib

__all__ = [
    "rotate_quant", "rotate_quant_out", "rank_projection", "rank_projection_out", "rank_projection_f16_out",
    "group_quant", "group_quant_out", "transform_f16", "transform_f16_out", "dynamic_asym_int4",
    "hadamard_rows", "dequantize", "w4a4_gemm", "w4a4_gemm_out", "prepare_rank_factors",
]

DEVICE = "cuda"
_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _p(t: Optional[Tensor]) -> Optional[ctypes.c_void_p]:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _workspace(nbytes: int, like: Tensor) -> Optional[Tensor]:
    return torch.empty(nbytes, dtype=torch.uint8, device=like.device) if nbytes else None


def _rank(w_t: Optional[Tensor]) -> int:
    return 0 if w_t is None else int(w_t.shape[0])


def _splits(partial: Optional[Tensor], k: int) -> int:
    return partial.shape[1] // k if partial is not None and k else 0


def _quant_outputs(x: Tensor, rows: int, group: int):
    n = x.shape[1]
    return (x.new_empty((rows, n // 2), dtype=torch.uint8),
            x.new_empty((rows, n // group), dtype=torch.float16),
            x.new_empty((rows, n // group), dtype=torch.float16))


# ------------------------------------------------------------- rotate_quant

def _rotate_quant_call(x, m, q, signs, v, w_t, prepared, rank_block, partial, group, dest_rows, rank_mode,
                       codes, scales, zeros, rotated) -> None:
    T, n = x.shape
    k = _rank(w_t)
    splits = _splits(partial, k)
    lib = _lib.load()
    ws_bytes = lib.narhip_rotate_quant_workspace(T, n, m, q, k, rank_block, int(partial is not None), splits,
                                                 int(prepared is not None), rank_mode)
    ws = _workspace(ws_bytes, x)
    _lib.check(lib.narhip_rotate_quant(
        _p(x), T, n, x.stride(0), m, q, _p(signs), k, rank_block, _p(v), _p(w_t), _p(prepared), _p(partial),
        splits, group, _p(codes), _p(scales), _p(zeros), _p(rotated), _p(dest_rows), rank_mode,
        _p(ws), ws_bytes, _stream(x)))


@torch.library.custom_op("narhip::rotate_quant_out", mutates_args=("codes", "scales", "zeros", "rotated"),
                         device_types=DEVICE)
def rotate_quant_out(x: Tensor, m: int, q: int, signs: Optional[Tensor], v: Optional[Tensor],
                     w_t: Optional[Tensor], prepared: Optional[Tensor], rank_block: int,
                     partial: Optional[Tensor], group: int, dest_rows: Optional[Tensor], rank_mode: int,
                     codes: Tensor, scales: Tensor, zeros: Tensor, rotated: Optional[Tensor]) -> None:
    """x' = (H_m (x) H_q) diag(signs) x - (x V) W''^T, INT4 over groups, into codes / scales /
    zeros (rows dest_rows[t] when given) and, when given, x' into ``rotated``."""
    _rotate_quant_call(x, m, q, signs, v, w_t, prepared, rank_block, partial, group, dest_rows, rank_mode,
                       codes, scales, zeros, rotated)


@rotate_quant_out.register_fake
def _(x, m, q, signs, v, w_t, prepared, rank_block, partial, group, dest_rows, rank_mode, codes, scales,
      zeros, rotated):
    return None


@torch.library.custom_op("narhip::rotate_quant", mutates_args=(), device_types=DEVICE)
def rotate_quant(x: Tensor, m: int, q: int, signs: Optional[Tensor], v: Optional[Tensor],
                 w_t: Optional[Tensor], prepared: Optional[Tensor], rank_block: int,
                 partial: Optional[Tensor], group: int, rank_mode: int) -> tuple[Tensor, Tensor, Tensor]:
    """rotate_quant_out into new (codes uint8 [T, n/2], scales fp16 [T, n/group], zeros)."""
    codes, scales, zeros = _quant_outputs(x, x.shape[0], group)
    _rotate_quant_call(x, m, q, signs, v, w_t, prepared, rank_block, partial, group, None, rank_mode,
                       codes, scales, zeros, None)
    return codes, scales, zeros


@rotate_quant.register_fake
def _(x, m, q, signs, v, w_t, prepared, rank_block, partial, group, rank_mode):
    return _quant_outputs(x, x.shape[0], group)


# ---------------------------------------------------------- rank projection

def _projection_call(x, v, prepared, k, rank_mode, partial) -> None:
    T, n = x.shape
    _lib.check(_lib.load().narhip_rank_projection(_p(x), T, n, x.stride(0), _p(v), _p(prepared), k,
                                                  partial.shape[1] // k, _p(partial), rank_mode, _stream(x)))


@torch.library.custom_op("narhip::rank_projection_out", mutates_args=("partial",), device_types=DEVICE)
def rank_projection_out(x: Tensor, v: Optional[Tensor], prepared: Optional[Tensor], k: int, rank_mode: int,
                        partial: Tensor) -> None:
    """partial[t, s*k + r] = sum over channel split s of x[t, i] v[i, r] (Kernel A)."""
    _projection_call(x, v, prepared, k, rank_mode, partial)


@rank_projection_out.register_fake
def _(x, v, prepared, k, rank_mode, partial):
    return None


@torch.library.custom_op("narhip::rank_projection", mutates_args=(), device_types=DEVICE)
def rank_projection(x: Tensor, v: Optional[Tensor], prepared: Optional[Tensor], k: int, splits: int,
                    rank_mode: int) -> Tensor:
    """rank_projection_out into a new fp32 [T, splits*k]."""
    partial = x.new_empty((x.shape[0], splits * k), dtype=torch.float32)
    _projection_call(x, v, prepared, k, rank_mode, partial)
    return partial


@rank_projection.register_fake
def _(x, v, prepared, k, splits, rank_mode):
    return x.new_empty((x.shape[0], splits * k), dtype=torch.float32)


@torch.library.custom_op("narhip::rank_projection_f16_out", mutates_args=("partial",), device_types=DEVICE)
def rank_projection_f16_out(x: Tensor, v: Tensor, partial: Tensor) -> None:
    """fp16 rows: partial[t, s*k + r] = RN32(exact sum over split s of x[t, i] v[i, r])."""
    T, n = x.shape
    k = int(v.shape[1])
    _lib.check(_lib.load().narhip_rank_projection_f16(_p(x), T, n, x.stride(0), _p(v), k, partial.shape[1] // k,
                                                      _p(partial), _stream(x)))


@rank_projection_f16_out.register_fake
def _(x, v, partial):
    return None


# --------------------------------------------------------------- group_quant

def _group_quant_call(x, partial, w_t, prepared, m, q, group, rank_mode, codes, scales, zeros) -> None:
    T, n = x.shape
    k = _rank(w_t)
    splits = _splits(partial, k)
    lib = _lib.load()
    ws_bytes = lib.narhip_rotate_quant_workspace(T, n, m, q, k, n, 1, splits, int(prepared is not None),
                                                 rank_mode)
    ws = _workspace(ws_bytes, x)
    _lib.check(lib.narhip_group_quant(_p(x), T, n, x.stride(0), m, q, _p(partial), splits, k, _p(w_t),
                                      _p(prepared), group, _p(codes), _p(scales), _p(zeros), rank_mode, _p(ws),
                                      ws_bytes, _stream(x)))


@torch.library.custom_op("narhip::group_quant_out", mutates_args=("codes", "scales", "zeros"),
                         device_types=DEVICE)
def group_quant_out(x: Tensor, partial: Optional[Tensor], w_t: Optional[Tensor], prepared: Optional[Tensor],
                    m: int, q: int, group: int, rank_mode: int, codes: Tensor, scales: Tensor,
                    zeros: Tensor) -> None:
    """Kernel B: rotate, fold the split partials into u, subtract u W''^T, quantize."""
    _group_quant_call(x, partial, w_t, prepared, m, q, group, rank_mode, codes, scales, zeros)


@group_quant_out.register_fake
def _(x, partial, w_t, prepared, m, q, group, rank_mode, codes, scales, zeros):
    return None


@torch.library.custom_op("narhip::group_quant", mutates_args=(), device_types=DEVICE)
def group_quant(x: Tensor, partial: Optional[Tensor], w_t: Optional[Tensor], prepared: Optional[Tensor],
                m: int, q: int, group: int, rank_mode: int) -> tuple[Tensor, Tensor, Tensor]:
    """group_quant_out into new outputs."""
    codes, scales, zeros = _quant_outputs(x, x.shape[0], group)
    _group_quant_call(x, partial, w_t, prepared, m, q, group, rank_mode, codes, scales, zeros)
    return codes, scales, zeros


@group_quant.register_fake
def _(x, partial, w_t, prepared, m, q, group, rank_mode):
    return _quant_outputs(x, x.shape[0], group)


# ------------------------------------------------------------- transform_f16

def _transform_f16_call(x, w_t, v, partial, had_q, out) -> None:
    T, n = x.shape
    k = _rank(w_t)
    splits = _splits(partial, k)
    lib = _lib.load()
    ws_bytes = lib.narhip_transform_f16_workspace(T, n, k)
    ws = _workspace(ws_bytes, x)
    _lib.check(lib.narhip_transform_f16(_p(x), T, n, x.stride(0), had_q, _p(v) if k else None,
                                        _p(partial) if k else None, splits, _p(w_t), k, _p(out), _p(ws),
                                        ws_bytes, _stream(x)))


@torch.library.custom_op("narhip::transform_f16_out", mutates_args=("out",), device_types=DEVICE)
def transform_f16_out(x: Tensor, w_t: Optional[Tensor], v: Optional[Tensor], partial: Optional[Tensor],
                      had_q: int, out: Tensor) -> None:
    """fp16 rows -> fp16: Hadamard blocks of had_q, minus u W''^T, u from partial or from v."""
    _transform_f16_call(x, w_t, v, partial, had_q, out)


@transform_f16_out.register_fake
def _(x, w_t, v, partial, had_q, out):
    return None


@torch.library.custom_op("narhip::transform_f16", mutates_args=(), device_types=DEVICE)
def transform_f16(x: Tensor, w_t: Optional[Tensor], v: Optional[Tensor], partial: Optional[Tensor],
                  had_q: int) -> Tensor:
    """transform_f16_out into a new fp16 [T, n]."""
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    _transform_f16_call(x, w_t, v, partial, had_q, out)
    return out


@transform_f16.register_fake
def _(x, w_t, v, partial, had_q):
    return torch.empty(x.shape, dtype=torch.float16, device=x.device)


# ------------------------------------------------------------------- hooks

def _int4_tuple_like(x: Tensor, group_size: int):
    n = x.shape[-1]
    lead = tuple(x.shape[:-1])
    groups = n // group_size
    return (torch.empty(x.shape, dtype=x.dtype, device=x.device),
            x.new_empty(lead + (groups,), dtype=torch.float16),
            x.new_empty(lead + (groups,), dtype=torch.float16),
            x.new_empty(lead + (groups, group_size), dtype=torch.uint8))


@torch.library.custom_op("narhip::dynamic_asym_int4", mutates_args=(), device_types=DEVICE)
def dynamic_asym_int4(x: Tensor, group_size: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(deq in x.dtype and x's shape, scale fp16 [..., G], zero fp16 [..., G], codes uint8 [..., G, b]),
    nar/experiment.py:158-184."""
    xc = x.contiguous()
    n = x.shape[-1]
    rows = xc.numel() // n if n else 0
    deq, scales, zeros, codes = _int4_tuple_like(xc, group_size)
    _lib.check(_lib.load().narhip_dynamic_asym_int4(_p(xc), _DTYPE_CODE[x.dtype], rows, n, group_size,
                                                    _p(codes), _p(scales), _p(zeros), _p(deq), _stream(x)))
    return deq, scales, zeros, codes


@dynamic_asym_int4.register_fake
def _(x, group_size):
    return _int4_tuple_like(x, group_size)


def _rotated_tuple_like(x: Tensor, group: int):
    T, n = x.shape
    return (x.new_empty((T, n), dtype=torch.float32),
            x.new_empty((T, n // group), dtype=torch.float16),
            x.new_empty((T, n // group), dtype=torch.float16),
            x.new_empty((T, n), dtype=torch.uint8))


@torch.library.custom_op("narhip::rotate_dynamic_asym_int4", mutates_args=(), device_types=DEVICE)
def rotate_dynamic_asym_int4(x: Tensor, m: int, q: int, signs: Optional[Tensor], v: Optional[Tensor],
                             w_t: Optional[Tensor], rank_block: int, group: int,
                             rank_mode: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """dynamic_asym_int4's tuple (deq fp32 [T, n], scale fp16 [T, n/group], zero, codes uint8 [T, n])
    of x' = (H_m (x) H_q) diag(signs) x - (x V) W''^T for bf16 rows x [T, n]."""
    T, n = x.shape
    k = _rank(w_t)
    deq, scales, zeros, codes = _rotated_tuple_like(x, group)
    lib = _lib.load()
    ws_bytes = lib.narhip_rotate_dynamic_asym_int4_workspace(T, n, m, q, k, rank_block, group, rank_mode)
    ws = _workspace(ws_bytes, x)
    _lib.check(lib.narhip_rotate_dynamic_asym_int4(_p(x), T, n, x.stride(0), m, q, _p(signs), k, rank_block, _p(v),
                                                   _p(w_t), group, _p(codes), _p(scales), _p(zeros), _p(deq),
                                                   rank_mode, _p(ws), ws_bytes, _stream(x)))
    return deq, scales, zeros, codes


@rotate_dynamic_asym_int4.register_fake
def _(x, m, q, signs, v, w_t, rank_block, group, rank_mode):
    return _rotated_tuple_like(x, group)


@torch.library.custom_op("narhip::hadamard_rows", mutates_args=(), device_types=DEVICE)
def hadamard_rows(x: Tensor, m: int, q: int, signs: Optional[Tensor]) -> Tensor:
    """fp32 [R, n] = (H_m (x) H_q) diag(signs) x of bf16 rows [R, n], n = m q."""
    R, n = x.shape
    out = x.new_empty((R, n), dtype=torch.float32)
    _lib.check(_lib.load().narhip_hadamard_rows(_p(x), R, n, x.stride(0), m, q, _p(signs), _p(out), _stream(x)))
    return out


@hadamard_rows.register_fake
def _(x, m, q, signs):
    return x.new_empty(x.shape, dtype=torch.float32)


# -------------------------------------------------------- dequantize, W4A4

@torch.library.custom_op("narhip::dequantize", mutates_args=(), device_types=DEVICE)
def dequantize(codes: Tensor, scales: Tensor, zeros: Tensor, n: int, group: int) -> Tensor:
    """fp32 [rows, n] = code * scale + zero of packed INT4 rows."""
    rows = codes.shape[0]
    out = codes.new_empty((rows, n), dtype=torch.float32)
    _lib.check(_lib.load().narhip_dequantize(_p(codes), _p(scales), _p(zeros), rows, n, group, _p(out),
                                             _stream(codes)))
    return out


@dequantize.register_fake
def _(codes, scales, zeros, n, group):
    return codes.new_empty((codes.shape[0], n), dtype=torch.float32)


def _w4a4_call(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group, out) -> None:
    T, half = a_codes.shape
    O = w_codes.shape[0]
    n = 2 * half
    lib = _lib.load()
    ws_bytes = lib.narhip_w4a4_workspace(T, O, n)
    ws = _workspace(ws_bytes, a_codes)
    _lib.check(lib.narhip_w4a4_gemm(_p(a_codes), _p(a_scales), _p(a_zeros), T, _p(w_codes), _p(w_scales),
                                    _p(w_zeros), O, n, group, _p(out), out.stride(0), _p(ws), ws_bytes,
                                    _stream(a_codes)))


@torch.library.custom_op("narhip::w4a4_gemm_out", mutates_args=("out",), device_types=DEVICE)
def w4a4_gemm_out(a_codes: Tensor, a_scales: Tensor, a_zeros: Tensor, w_codes: Tensor, w_scales: Tensor,
                  w_zeros: Tensor, group: int, out: Tensor) -> None:
    """out fp32 [T, O] = dequant(A) dequant(W)^T of two packed group-asymmetric INT4 operands."""
    _w4a4_call(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group, out)


@w4a4_gemm_out.register_fake
def _(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group, out):
    return None


@torch.library.custom_op("narhip::w4a4_gemm", mutates_args=(), device_types=DEVICE)
def w4a4_gemm(a_codes: Tensor, a_scales: Tensor, a_zeros: Tensor, w_codes: Tensor, w_scales: Tensor,
              w_zeros: Tensor, group: int) -> Tensor:
    """w4a4_gemm_out into a new fp32 [T, O]."""
    out = a_codes.new_empty((a_codes.shape[0], w_codes.shape[0]), dtype=torch.float32)
    _w4a4_call(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group, out)
    return out


@w4a4_gemm.register_fake
def _(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group):
    return a_codes.new_empty((a_codes.shape[0], w_codes.shape[0]), dtype=torch.float32)


# ------------------------------------------------------------ factor terms

def _prepared_bytes(n: int, k: int) -> int:
    nbytes = _lib.load().narhip_rank_factors_bytes(n, k)
    if nbytes == 0:
        raise ValueError(f"no prepared layout for n={n}, k={k}")
    return nbytes


@torch.library.custom_op("narhip::prepare_rank_factors", mutates_args=(), device_types=DEVICE)
def prepare_rank_factors(v: Optional[Tensor], w_t: Optional[Tensor], n: int, k: int) -> Tensor:
    """V and W''^T as exact bf16 term triples in the MFMA operand layouts (uint8 buffer); a
    factor passed as None leaves its half of the buffer unwritten."""
    ref = v if v is not None else w_t
    out = ref.new_empty(_prepared_bytes(n, k), dtype=torch.uint8)
    _lib.check(_lib.load().narhip_prepare_rank_factors(_p(v), _p(w_t), n, k, _p(out), out.numel(), _stream(ref)))
    return out


@prepare_rank_factors.register_fake
def _(v, w_t, n, k):
    ref = v if v is not None else w_t
    return ref.new_empty(_prepared_bytes(n, k), dtype=torch.uint8)
