"""Drop-in for nar/kernels/r4_fused_v3.py on MI355X (HIP kernels in libnarhip.so).

Same names and signatures as the reference module (nar/kernels/r4_fused_v3.py:
39-271).  ``launch_projection_dot`` takes the reference's stacked bf16 (or, for
fp16 rows, fp16) factor terms (y_padded [TERMS*n, KP]), rebuilds the fp32
factor they represent and runs narhip's Kernel A (bf16 MFMA, or fp64 VALU for
fp16 rows); ``launch_nar`` / ``launch_hadamard`` run
narhip's Kernel B.  The Triton tile dataclasses and config lists are kept so
that the reference's verify-then-time harnesses run unchanged: the HIP kernels
pick their own tiles, so ``block_t``/``num_warps``/``num_stages``/``use_dot``
are accepted and ignored, and ``ProjectionConfig.splits`` still sets the
partial layout partial[t, s*k + r].
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from narhip import ops
from narhip.factors import IdentityCache, cached_prepared

from .r4_fused_v2 import (GROUP, PackedInt4, allocate_outputs, allocate_partial,  # noqa: F401
                          dequantize, reduce_partial, unpack)

__all__ = ["GROUP", "PackedInt4", "allocate_outputs", "allocate_partial", "dequantize",
           "reduce_partial", "unpack", "ProjectionConfig", "TileConfig",
           "PROJECTION_CONFIGS", "TILE_CONFIGS", "padded_rank",
           "projection_cublas_fp32_out", "projection_cublas_fp32_out_split",
           "launch_projection_dot", "launch_nar", "launch_hadamard"]


def padded_rank(k: int) -> int:
    """The reference pads the rank to at least 16 columns (a power of two)."""
    return max(16, 1 << (k - 1).bit_length())


def _mm_fp32_out(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return torch.mm(x, y, out_dtype=torch.float32)


def cublas_fp32_out_supported() -> bool:
    try:
        a = torch.zeros((16, 16), dtype=torch.bfloat16, device="cuda")
        _mm_fp32_out(a, a)
        return True
    except (TypeError, RuntimeError):
        return False


def projection_cublas_fp32_out(x: torch.Tensor, y_prime_bf16: torch.Tensor,
                               partial: torch.Tensor) -> torch.Tensor:
    return _mm_fp32_out(x, y_prime_bf16)


def projection_cublas_fp32_out_split(x: torch.Tensor, terms: tuple[torch.Tensor, ...],
                                     partial: torch.Tensor) -> torch.Tensor:
    result = _mm_fp32_out(x, terms[0])
    for term in terms[1:]:
        result.add_(_mm_fp32_out(x, term))
    return result


@dataclass(frozen=True)
class ProjectionConfig:
    block_t: int
    block_d: int
    splits: int
    num_warps: int
    num_stages: int

    def label(self) -> str:
        return (f"T{self.block_t}_D{self.block_d}_S{self.splits}"
                f"_w{self.num_warps}_s{self.num_stages}")


@dataclass(frozen=True)
class TileConfig:
    block_t: int
    num_warps: int
    num_stages: int
    use_dot: bool = False

    def label(self) -> str:
        return (f"T{self.block_t}_w{self.num_warps}_s{self.num_stages}"
                f"{'_dot' if self.use_dot else ''}")


PROJECTION_CONFIGS = tuple(
    ProjectionConfig(block_t, block_d, splits, warps, stages)
    for block_t, block_d, warps, stages in (
        (16, 64, 4, 4), (16, 128, 4, 4), (16, 256, 8, 3),
        (32, 64, 4, 4), (32, 128, 8, 3), (32, 256, 8, 3),
        (64, 64, 8, 3), (64, 128, 8, 3),
    )
    for splits in (1, 2, 4)
)

TILE_CONFIGS = tuple(
    TileConfig(block_t, warps, stages)
    for block_t, warps, stages in (
        (1, 4, 1), (2, 4, 2), (4, 4, 2), (4, 8, 2),
        (8, 4, 2), (8, 8, 3), (16, 8, 3), (32, 8, 2), (64, 8, 2),
    )
) + tuple(TileConfig(block_t, warps, stages, use_dot=True)
          for block_t, warps, stages in ((16, 8, 3), (32, 8, 2), (64, 8, 2)))

_FACTOR_FROM_TERMS = IdentityCache()


def _factor_from_terms(y_padded: torch.Tensor, n: int, k: int, terms: int) -> torch.Tensor:
    """Sum of the first `terms` stacked bf16 terms -> fp32 [n, k] (exact for <= 3 terms)."""
    def make() -> torch.Tensor:
        kp = y_padded.shape[1]
        stacked = y_padded.reshape(-1, n, kp)[:terms, :, :k].float()
        v = stacked[0].clone()
        for t in range(1, terms):
            v += stacked[t]
        return v.contiguous()
    return _FACTOR_FROM_TERMS.get((y_padded,), (n, k, terms), make)


def launch_projection_dot(x: torch.Tensor, y_padded: torch.Tensor, partial: torch.Tensor,
                          k: int, config: ProjectionConfig, terms: int) -> torch.Tensor:
    tokens, n = x.shape
    if n % config.splits:
        raise ValueError(f"{n} channels do not divide into {config.splits} splits")
    if partial.shape != (tokens, config.splits * k):
        raise ValueError(f"partial must be [{tokens}, {config.splits * k}]")
    v = _factor_from_terms(y_padded, n, k, terms)
    if x.dtype == torch.float16:
        # E28 feeds fp16 rows with TERMS = 2 fp16 factor terms
        # (quarot-llama3/nar_r4_kernel.py:267,272): fp64 VALU projection.
        return ops.rank_projection_f16(x, v, partial)
    if n % (128 * config.splits) == 0:
        prep = cached_prepared(v, None, n, k)
        return ops.rank_projection(x, v, partial, ops.RANK_MFMA, prepared=prep)
    return ops.rank_projection(x, v, partial, ops.RANK_EXACT)


def launch_nar(x: torch.Tensor, w_h_t_fp32: torch.Tensor, outputs: PackedInt4,
               partial: torch.Tensor, k: int, tile: TileConfig,
               *, group: int = GROUP, hadamard: tuple[int, int] = (1, GROUP),
               rank_mode: int = ops.RANK_AUTO) -> None:
    tokens, n = x.shape
    if w_h_t_fp32.shape != (k, n):
        raise ValueError(f"w_h_t_fp32 must be [{k}, {n}]")
    prep = cached_prepared(None, w_h_t_fp32, n, k) if rank_mode != ops.RANK_EXACT and k >= 16 else None
    ops.group_quant(x, partial, w_h_t_fp32, outputs.codes, outputs.scales, outputs.zeros,
                    hadamard=hadamard, group=group, prepared=prep, rank_mode=rank_mode)


def launch_hadamard(x: torch.Tensor, outputs: PackedInt4, tile: TileConfig,
                    *, group: int = GROUP, hadamard: tuple[int, int] = (1, GROUP)) -> None:
    ops.rotate_quant(x, hadamard=hadamard, group=group,
                     codes=outputs.codes, scales=outputs.scales, zeros=outputs.zeros)
