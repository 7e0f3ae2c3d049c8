"""The reference's PyTorch CPU op sequence for the path, restated (baseline only).

TEST INFRASTRUCTURE ONLY: bench.py times this as the CPU baseline; nothing in
the product calls it.  It performs the same tensor operations the reference
performs on the CPU, in the same order:
  full_hadamard_rows        nar/activation_experiments.py:188-217
    (_fast_walsh_hadamard   nar/extended_experiment.py:443-456, torch.cat stages,
     Paley factor as a dense torch matmul)
  rank-k row form           quarot-llama3/nar_r4_kernel.py:190-202 (u = x @ Y', h - u @ W''^T)
  dynamic_asym_int4         nar/experiment.py:158-184
  nibble packing            nar/kernels/r4_fused_v2.py:80-92
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import oracle as O


def fwht(x: torch.Tensor) -> torch.Tensor:
    n = x.shape[-1]
    shape = x.shape
    y = x.reshape(-1, n)
    width = 1
    while width < n:
        blocks = y.reshape(-1, n // (2 * width), 2, width)
        y = torch.cat((blocks[:, :, 0, :] + blocks[:, :, 1, :], blocks[:, :, 0, :] - blocks[:, :, 1, :]), dim=-1)
        y = y.reshape(-1, n)
        width *= 2
    return (y / math.sqrt(n)).reshape(shape)


def hadamard_rows(x: torch.Tensor, m: int, q: int) -> torch.Tensor:
    if m == 1:
        return fwht(x.reshape(-1, x.shape[-1] // q, q)).reshape_as(x)
    hm = torch.from_numpy(O.paley(m).astype(np.float32)) / math.sqrt(m)
    factored = fwht(x.reshape(-1, m, q))
    return (factored.transpose(1, 2) @ hm.T).transpose(1, 2).reshape_as(x)


def dynamic_asym_int4(x: torch.Tensor, b: int):
    xg = x.float().reshape(*x.shape[:-1], x.shape[-1] // b, b)
    lo = xg.amin(dim=-1, keepdim=True)
    hi = xg.amax(dim=-1, keepdim=True)
    raw = (hi - lo) / 15
    s16 = torch.where(raw > 0, raw, torch.ones_like(raw)).to(torch.float16)
    s16 = torch.where(s16 > 0, s16, torch.ones_like(s16))
    z16 = lo.to(torch.float16)
    q = torch.round((xg - z16.float()) / s16.float()).clamp_(0, 15)
    return q.to(torch.uint8).reshape_as(x), s16.squeeze(-1), z16.squeeze(-1)


def run(x_bits: np.ndarray, m: int, q: int, v: np.ndarray | None, w_t: np.ndarray | None,
        group: int, rank_block: int | None = None):
    """bf16 bits [T, n] -> (packed codes, fp16 scales, fp16 zeros) on the CPU."""
    x = torch.from_numpy(O.bf16_to_f32(x_bits))
    n = x.shape[1]
    h = hadamard_rows(x, m, q)
    if v is not None:
        nb = n if rank_block is None else rank_block
        vt, wt = torch.from_numpy(v), torch.from_numpy(w_t)
        if nb == n:
            h = h - (x @ vt) @ wt
        else:
            blocks = n // nb
            xb = x.reshape(-1, blocks, nb)
            u = torch.einsum("tbi,bik->tbk", xb, vt.reshape(blocks, nb, -1))
            corr = torch.einsum("tbk,bki->tbi", u, wt.reshape(-1, blocks, nb).transpose(0, 1))
            h = h - corr.reshape_as(h)
    codes, s16, z16 = dynamic_asym_int4(h, group)
    packed = codes[:, 0::2] | (codes[:, 1::2] << 4)
    return packed, s16, z16
