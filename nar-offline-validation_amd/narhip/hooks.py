"""GPU drop-ins for the hook-side functions of the path.

The reference's fake-quant hooks (KVQuantAttention, nar/experiment.py:887-910;
ActivationQuantHooks.quantize, nar/activation_experiments.py:603-606; the E14
RuntimeHooks V path and the E17 DownHooks) rotate a tensor with
``full_hadamard_rows`` and then call ``dynamic_asym_int4``.  These functions
keep those names, signatures, return layouts and exceptions, and run on the
HIP kernels of libnarhip.so:

  dynamic_asym_int4(x, group_size) -> (deq, scale16, zero16, codes)
      nar/experiment.py:158-184.  deq in x.dtype and x's shape; scale16 and
      zero16 fp16 [..., G]; codes uint8 [..., G, group_size] (one per byte).
  full_hadamard_rows(x, signs) -> (H_m (x) H_q) diag(signs) x, x's shape
      nar/activation_experiments.py:188-217, for widths 28 * 2^j, 12 * 2^j,
      20 * 2^j (j = 7, 8), the Qwen3 widths 68 * 2^j, 76 * 2^j, 200 * 2^j
      (up to 32768 channels) and 2^j <= 8192.  The kernels read bf16 rows: x must be bf16,
      or fp32 holding bf16 values (the hooks pass ``value.float()`` of a bf16
      model).
  rotate_dynamic_asym_int4(x, group_size, *, signs=None, v=None, w_t=None,
                           block=None, rank_block=None)
      both in one call -- full-row or per-block (per-head) Hadamard, optional
      rank-k term x' = Hx + U(V^T x) over the row or per block (w_t = W''^T =
      -U^T) -- returning dynamic_asym_int4's tuple of x'.

Device tensors only; there is no CPU path.
"""

from __future__ import annotations

import torch

from .ops import RANK_AUTO, _ops, _require, hadamard_factors

_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _group_view_check(n: int, group_size: int) -> None:
    if n % group_size:
        raise ValueError(f"last dimension {n} is not divisible by group size {group_size}")


def dynamic_asym_int4(x: torch.Tensor, group_size: int):
    """Fake-quantize with one fp16 scale and fp16 zero per group of the last dimension."""
    if not x.is_cuda:
        raise ValueError("dynamic_asym_int4 (narhip) takes device tensors")
    if x.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {x.dtype}")
    _group_view_check(x.shape[-1], group_size)
    return _ops.dynamic_asym_int4(x, group_size)


def _as_bf16_rows(x: torch.Tensor) -> torch.Tensor:
    n = x.shape[-1]
    if x.dtype == torch.bfloat16:
        xb = x
    elif x.dtype == torch.float32:
        xb = x.to(torch.bfloat16)
        if not torch.equal(xb.float(), x):
            raise ValueError("full_hadamard_rows (narhip) reads bf16 rows: x holds values that are not bf16")
    else:
        raise ValueError(f"unsupported dtype {x.dtype}")
    return xb.contiguous().view(-1, n)


def _signs_f32(signs: torch.Tensor | None, n: int, device: torch.device) -> torch.Tensor | None:
    if signs is None:
        return None
    s = signs.to(device=device, dtype=torch.float32).contiguous().view(-1)
    if s.numel() != n:
        raise ValueError(f"signs must have {n} entries")
    return s


def full_hadamard_rows(x: torch.Tensor, signs: torch.Tensor | None) -> torch.Tensor:
    """(H_m (x) H_q) diag(signs) x along the last dimension, fp32 out, x's shape."""
    if not x.is_cuda:
        raise ValueError("full_hadamard_rows (narhip) takes device tensors")
    n = x.shape[-1]
    m, q = hadamard_factors(n)
    xb = _as_bf16_rows(x)
    return _ops.hadamard_rows(xb, m, q, _signs_f32(signs, n, x.device)).view(x.shape)


def rotate_dynamic_asym_int4(x: torch.Tensor, group_size: int, *, signs: torch.Tensor | None = None,
                             v: torch.Tensor | None = None, w_t: torch.Tensor | None = None,
                             block: int | None = None, rank_block: int | None = None,
                             rank_mode: int = RANK_AUTO):
    """dynamic_asym_int4 of x' = H diag(signs) x + U (V^T x); the tuple of x' in fp32.

    H is full_hadamard_rows' construction over the last dimension (block None)
    or the block-diagonal H_block (e.g. block = head_dim: one H per head).  The
    rank term takes v fp32 [n, k] and w_t = W''^T = -U^T fp32 [k, n], over the
    whole row (rank_block None) or per block (rank_block = block: per-head
    factors stacked along n, k <= 8).  One kernel reads x once and writes the
    tuple for the block and per-head forms, the power-of-two widths and the
    Kronecker widths without a rank term (groups of 32, 64 or 128).
    """
    if not x.is_cuda:
        raise ValueError("rotate_dynamic_asym_int4 (narhip) takes device tensors")
    n = x.shape[-1]
    _group_view_check(n, group_size)
    if block is None:
        m, q = hadamard_factors(n)
    else:
        if n % block:
            raise ValueError(f"last dimension {n} is not a multiple of the Hadamard block {block}")
        m, q = 1, int(block)
    xb = _as_bf16_rows(x)
    k = 0 if w_t is None else int(w_t.shape[0])
    if k:
        if v is None:
            raise ValueError("the rank term needs v and w_t")
        _require(v, torch.float32, "v", x.device)
        _require(w_t, torch.float32, "w_t", x.device)
        if tuple(v.shape) != (n, k) or tuple(w_t.shape) != (k, n):
            raise ValueError(f"v must be [{n}, {k}] and w_t [{k}, {n}]")
    nb = n if rank_block is None else int(rank_block)
    deq, scale, zero, codes = _ops.rotate_dynamic_asym_int4(xb, m, q, _signs_f32(signs, n, x.device), v, w_t, nb,
                                                            group_size, rank_mode)
    lead = tuple(x.shape[:-1])
    groups = n // group_size
    return (deq.view(x.shape), scale.view(lead + (groups,)), zero.view(lead + (groups,)),
            codes.view(lead + (groups, group_size)))
