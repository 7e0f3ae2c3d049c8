"""Keyword-friendly wrappers of the narhip operators.

Each function checks its arguments the way the reference's launchers do
(``ValueError`` for dtype, device, shape and layout) and then calls the
registered ``torch.ops.narhip`` operator (narhip/library.py), which runs the
HIP kernels on the current stream of the tensors' device.  Outputs are
allocated here when the caller does not pass them (the reference's launchers
take them preallocated; both forms are supported).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from . import library  # noqa: F401  (registers torch.ops.narhip)

_ops = torch.ops.narhip

RANK_AUTO, RANK_EXACT, RANK_MFMA = _lib.RANK_AUTO, _lib.RANK_EXACT, _lib.RANK_MFMA


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require(t: torch.Tensor, dtype: torch.dtype, name: str, device: torch.device) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


QWEN3_PALEY_ORDERS = (20, 68, 76, 200)


def hadamard_factors(n: int) -> tuple[int, int]:
    """(m, q) with n = m*q in the dispatch order of full_hadamard_rows
    (nar/activation_experiments.py:188-217): 28 * 2^j first, then 12 * 2^j,
    then, for widths that are not a power of two, the Qwen3 Paley orders
    20, 68, 76 and 200 times 2^j, then a power of two.  The Kronecker
    kernels build m in {1, 12, 20, 28}; 68, 76 and 200 run as whole rows
    (hadamard_rows and the hooks' tuple, no rank term)."""
    def pow2(v: int) -> bool:
        return v >= 1 and not v & (v - 1)

    for m in (28, 12):
        q, r = divmod(n, m)
        if not r and pow2(q):
            return m, q
    if not pow2(n):
        for m in QWEN3_PALEY_ORDERS:
            q, r = divmod(n, m)
            if not r and pow2(q):
                return m, q
    if pow2(n):
        return 1, n
    raise ValueError(f"no frozen full-Hadamard construction for n={n}")


def paley(m: int) -> torch.Tensor:
    """The +-1 Paley factor the kernels use (int8 [m, m], host)."""
    out = torch.empty((m, m), dtype=torch.int8)
    _lib.check(_lib.load().narhip_paley(m, _p(out)))
    return out


def prepare_rank_factors(v: torch.Tensor | None, w_t: torch.Tensor | None, n: int, k: int) -> torch.Tensor:
    """V and W''^T as exact bf16 term triples in the MFMA layouts (uint8 buffer).

    Done once per factor set, like the reference's term padding in
    FoldedR4.from_factor / NARDownTransform.__init__."""
    ref = v if v is not None else w_t
    if ref is None:
        raise ValueError("pass v, w_t or both")
    dev = ref.device
    if v is not None:
        _require(v, torch.float32, "v", dev)
        if tuple(v.shape) != (n, k):
            raise ValueError(f"v must be [{n}, {k}], got {tuple(v.shape)}")
    if w_t is not None:
        _require(w_t, torch.float32, "w_t", dev)
        if tuple(w_t.shape) != (k, n):
            raise ValueError(f"w_t must be [{k}, {n}], got {tuple(w_t.shape)}")
    return _ops.prepare_rank_factors(v, w_t, n, k)


def rotate_quant(x: torch.Tensor, *, hadamard: tuple[int, int] = (1, 128),
                 signs: torch.Tensor | None = None,
                 v: torch.Tensor | None = None, w_t: torch.Tensor | None = None,
                 prepared: torch.Tensor | None = None,
                 rank_block: int | None = None,
                 partial: torch.Tensor | None = None,
                 group: int = 128,
                 codes: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                 zeros: torch.Tensor | None = None,
                 rotated: torch.Tensor | None = None,
                 dest_rows: torch.Tensor | None = None,
                 rank_mode: int = RANK_AUTO,
                 out_rows: int | None = None):
    """x' = H_s x - (x V) W^T, then dynamic asymmetric INT4 over groups of `group`.

    x: bf16 [T, n] (row stride a multiple of 8).  v: fp32 [n, k], w_t: fp32 [k, n].
    Returns (codes uint8 [R, n/2], scales fp16 [R, n/group], zeros fp16 [R, n/group]).
    """
    if x.dim() != 2:
        raise ValueError("x must be 2-D [tokens, n]")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"x must be bfloat16, got {x.dtype}")
    if not x.is_cuda:
        raise ValueError("x must be a GPU tensor")
    if x.stride(1) != 1:
        raise ValueError("x rows must be contiguous")
    dev = x.device
    T, n = x.shape
    m, q = hadamard
    k = 0 if w_t is None else int(w_t.shape[0])
    if k:
        _require(w_t, torch.float32, "w_t", dev)
        if v is not None:
            _require(v, torch.float32, "v", dev)
            if v.shape != (n, k):
                raise ValueError(f"v must be [{n}, {k}], got {tuple(v.shape)}")
        if w_t.shape != (k, n):
            raise ValueError(f"w_t must be [{k}, {n}], got {tuple(w_t.shape)}")
    if signs is not None:
        _require(signs, torch.float32, "signs", dev)
    if partial is not None:
        _require(partial, torch.float32, "partial", dev)
        if not k or partial.shape[0] != T or partial.shape[1] % k:
            raise ValueError("partial must be [tokens, splits*k]")
    nb = n if rank_block is None else int(rank_block)
    if rotated is not None:
        _require(rotated, torch.float32, "rotated", dev)
    if dest_rows is not None:
        _require(dest_rows, torch.int64, "dest_rows", dev)
    if codes is None and scales is None and zeros is None and rotated is None and dest_rows is None \
            and out_rows is None:
        return _ops.rotate_quant(x, m, q, signs, v, w_t, prepared, nb, partial, group, rank_mode)
    rows = T if out_rows is None else out_rows
    if codes is None:
        codes = torch.empty((rows, n // 2), dtype=torch.uint8, device=dev)
    if scales is None:
        scales = torch.empty((rows, n // group), dtype=torch.float16, device=dev)
    if zeros is None:
        zeros = torch.empty((rows, n // group), dtype=torch.float16, device=dev)
    for t, name, dt in ((codes, "codes", torch.uint8), (scales, "scales", torch.float16),
                        (zeros, "zeros", torch.float16)):
        _require(t, dt, name, dev)
    _ops.rotate_quant_out(x, m, q, signs, v, w_t, prepared, nb, partial, group, dest_rows, rank_mode,
                          codes, scales, zeros, rotated)
    return codes, scales, zeros


def rank_projection(x: torch.Tensor, v: torch.Tensor | None, partial: torch.Tensor,
                    rank_mode: int = RANK_AUTO, *, prepared: torch.Tensor | None = None,
                    k: int | None = None) -> torch.Tensor:
    """partial[t, s*k + r] = sum over channel split s of x[t, i] v[i, r]."""
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be bfloat16 with contiguous rows")
    dev = x.device
    if v is not None:
        _require(v, torch.float32, "v", dev)
        k = int(v.shape[1])
    if k is None:
        raise ValueError("rank k unknown: pass v or k")
    _require(partial, torch.float32, "partial", dev)
    T, n = x.shape
    if partial.shape[0] != T or partial.shape[1] % k:
        raise ValueError("partial must be [tokens, splits*k]")
    _ops.rank_projection_out(x, v, prepared, k, rank_mode, partial)
    return partial


def rank_projection_f16(x: torch.Tensor, v: torch.Tensor, partial: torch.Tensor) -> torch.Tensor:
    """fp16 rows: partial[t, s*k + r] = RN32(sum over channel split s of x[t, i] v[i, r]), fp64 sums."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a float16 [tokens, n] tensor with contiguous rows")
    if not x.is_cuda:
        raise ValueError("x must be a GPU tensor")
    dev = x.device
    _require(v, torch.float32, "v", dev)
    _require(partial, torch.float32, "partial", dev)
    T, n = x.shape
    k = int(v.shape[1])
    if v.shape[0] != n:
        raise ValueError(f"v must be [{n}, k], got {tuple(v.shape)}")
    if partial.shape[0] != T or partial.shape[1] % k:
        raise ValueError("partial must be [tokens, splits*k]")
    _ops.rank_projection_f16_out(x, v, partial)
    return partial


def transform_f16(x: torch.Tensor, w_t: torch.Tensor | None, *, v: torch.Tensor | None = None,
                  partial: torch.Tensor | None = None, had_q: int = 128,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 [tokens, n] -> fp16: Hadamard blocks of had_q, minus u W^T (E28's transform).

    u is folded from `partial` [tokens, splits*k] when given, else computed from
    v [n, k]; w_t is fp32 [k, n] (None: Hadamard blocks only).
    """
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a float16 [tokens, n] tensor with contiguous rows")
    if not x.is_cuda:
        raise ValueError("x must be a GPU tensor")
    dev = x.device
    T, n = x.shape
    k = 0 if w_t is None else int(w_t.shape[0])
    if k:
        _require(w_t, torch.float32, "w_t", dev)
        if w_t.shape[1] != n:
            raise ValueError(f"w_t must be [k, {n}], got {tuple(w_t.shape)}")
        if partial is not None:
            _require(partial, torch.float32, "partial", dev)
            if partial.shape[0] != T or partial.shape[1] % k:
                raise ValueError(f"partial must be [{T}, splits*{k}]")
        else:
            if v is None:
                raise ValueError("the rank term needs v or partial")
            _require(v, torch.float32, "v", dev)
            if tuple(v.shape) != (n, k):
                raise ValueError(f"v must be [{n}, {k}], got {tuple(v.shape)}")
    if out is None:
        return _ops.transform_f16(x, w_t, v, partial, had_q)
    _require(out, torch.float16, "out", dev)
    if tuple(out.shape) != (T, n):
        raise ValueError(f"out must be [{T}, {n}], got {tuple(out.shape)}")
    _ops.transform_f16_out(x, w_t, v, partial, had_q, out)
    return out


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """Unpacked codes uint8 [..., n] (0..15) -> packed [..., n/2], low nibble = even channel."""
    if codes.dtype != torch.uint8 or codes.shape[-1] % 2:
        raise ValueError("codes must be uint8 with an even last dimension")
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()


def w4a4_gemm(a_codes: torch.Tensor, a_scales: torch.Tensor, a_zeros: torch.Tensor,
              w_codes: torch.Tensor, w_scales: torch.Tensor, w_zeros: torch.Tensor, *,
              group: int = 128, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [T, O] = dequant(A) @ dequant(W)^T for two packed INT4 operands (group-asymmetric).

    a_codes uint8 [T, n/2], a_scales / a_zeros fp16 [T, n/group]; w_* likewise
    with O rows (weights quantized along their input dimension).
    """
    dev = a_codes.device
    if not a_codes.is_cuda:
        raise ValueError("operands must be GPU tensors")
    T, half = a_codes.shape
    O = w_codes.shape[0]
    n = 2 * half
    for t, dt, shape, name in ((a_codes, torch.uint8, (T, half), "a_codes"), (w_codes, torch.uint8, (O, half), "w_codes"),
                               (a_scales, torch.float16, (T, n // group), "a_scales"),
                               (a_zeros, torch.float16, (T, n // group), "a_zeros"),
                               (w_scales, torch.float16, (O, n // group), "w_scales"),
                               (w_zeros, torch.float16, (O, n // group), "w_zeros")):
        _require(t, dt, name, dev)
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")
    if out is None:
        return _ops.w4a4_gemm(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group)
    _require(out, torch.float32, "out", dev)
    if tuple(out.shape) != (T, O):
        raise ValueError(f"out must be [{T}, {O}], got {tuple(out.shape)}")
    _ops.w4a4_gemm_out(a_codes, a_scales, a_zeros, w_codes, w_scales, w_zeros, group, out)
    return out


def group_quant(x: torch.Tensor, partial: torch.Tensor | None, w_t: torch.Tensor | None,
                codes: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, *,
                hadamard: tuple[int, int] = (1, 128), group: int = 128,
                prepared: torch.Tensor | None = None, rank_mode: int = RANK_AUTO) -> None:
    """Kernel B: rotate, fold the split partials, subtract u W^T, quantize."""
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be bfloat16 with contiguous rows")
    dev = x.device
    T, n = x.shape
    k = 0 if w_t is None else int(w_t.shape[0])
    if k:
        _require(w_t, torch.float32, "w_t", dev)
        if partial is None:
            raise ValueError("the rank term needs the projection partials")
        _require(partial, torch.float32, "partial", dev)
        if partial.shape[0] != T or partial.shape[1] % k:
            raise ValueError(f"partial must be [{T}, splits*{k}]")
    for t, name, dt in ((codes, "codes", torch.uint8), (scales, "scales", torch.float16),
                        (zeros, "zeros", torch.float16)):
        _require(t, dt, name, dev)
    m, q = hadamard
    _ops.group_quant_out(x, partial if k else None, w_t, prepared, m, q, group, rank_mode, codes, scales, zeros)


def dequantize(codes: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, n: int,
               group: int) -> torch.Tensor:
    dev = codes.device
    _require(codes, torch.uint8, "codes", dev)
    _require(scales, torch.float16, "scales", dev)
    _require(zeros, torch.float16, "zeros", dev)
    return _ops.dequantize(codes, scales, zeros, n, group)


def mfma_probe(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """One v_mfma_f32_16x16x32_bf16 on per-lane operands a, b (bf16 [64, 8]) -> fp32 [64, 4]."""
    dev = a.device
    _require(a, torch.bfloat16, "a", dev)
    _require(b, torch.bfloat16, "b", dev)
    d = torch.empty((64, 4), dtype=torch.float32, device=dev)
    _lib.check(_lib.load().narhip_mfma_probe(_p(a), _p(b), _p(d), _stream(dev)))
    return d


def sqrt_f32(v: int) -> float:
    return float(torch.tensor(math.sqrt(v), dtype=torch.float32))
