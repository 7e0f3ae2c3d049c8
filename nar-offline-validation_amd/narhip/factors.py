"""Host-side factor bookkeeping shared by the drop-in modules.

The reference prepares its factor terms once per factor set (FoldedR4.from_factor,
nar/fold_signed_permutation.py:70-114; NARDownTransform.__init__,
quarot-llama3/nar_r4_kernel.py:225-243).  Call sites of the launcher API pass
the raw fp32 factors on every call, so the derived device buffers (the [n, k]
transpose of Y'^T and the prepared MFMA terms) are cached per source tensor,
keyed by storage pointer, shape and version counter (an in-place update of the
factor invalidates the entry).
"""

from __future__ import annotations

import torch

from . import ops

_TRANSPOSE: dict[tuple, torch.Tensor] = {}
_PREPARED: dict[tuple, torch.Tensor] = {}
_MAX_ENTRIES = 64


def _key(t: torch.Tensor | None) -> tuple:
    if t is None:
        return (None,)
    return (t.data_ptr(), tuple(t.shape), t.dtype, str(t.device), t._version)


def _remember(cache: dict, key: tuple, value: torch.Tensor) -> torch.Tensor:
    if len(cache) >= _MAX_ENTRIES:
        cache.pop(next(iter(cache)))
    cache[key] = value
    return value


def cached_transpose(y_t: torch.Tensor) -> torch.Tensor:
    """fp32 [k, n] -> contiguous fp32 [n, k]."""
    key = _key(y_t)
    hit = _TRANSPOSE.get(key)
    if hit is not None:
        return hit
    return _remember(_TRANSPOSE, key, y_t.float().t().contiguous())


def cached_prepared(v: torch.Tensor | None, w_t: torch.Tensor | None, n: int, k: int) -> torch.Tensor:
    """Prepared MFMA factor terms for (v, w_t); either half may be absent."""
    key = (_key(v), _key(w_t), n, k)
    hit = _PREPARED.get(key)
    if hit is not None:
        return hit
    vv = None if v is None else v.float().contiguous()
    ww = None if w_t is None else w_t.float().contiguous()
    return _remember(_PREPARED, key, ops.prepare_rank_factors(vv, ww, n, k))


def clear() -> None:
    _TRANSPOSE.clear()
    _PREPARED.clear()
