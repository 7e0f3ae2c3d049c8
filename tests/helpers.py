"""Shared helpers for the parity tests (host <-> device, oracle runs)."""

from __future__ import annotations

import numpy as np

from oracle import oracle as O


def to_dev_bf16(bits: np.ndarray, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def to_dev_f32(a: np.ndarray | None, device="cuda"):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def f16_bits(t) -> np.ndarray:
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_for(w, rows: np.ndarray | None = None):
    """Oracle rotated rows and quantization for workload w (optionally a row subset)."""
    x = O.bf16_to_f32(w.x if rows is None else w.x[rows])
    m, q = w.hadamard
    rot = O.rotate(x, m, q, v=w.v, wt=w.w_t, rank_block=w.rank_block)
    return rot, O.quant(rot, w.group)
