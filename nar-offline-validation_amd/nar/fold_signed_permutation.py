"""Drop-in for nar/fold_signed_permutation.py: the signed-permutation fold of NAR R4.

Same names and behaviour as the reference module (nar/fold_signed_permutation.py:
27-152): ``source_for_target``, ``signed_permute_rows``,
``block_hadamard_columns``, ``FoldedR4`` (``from_factor``, ``q_unfolded``,
``apply``, ``save``; plus ``load``), ``fold_swiglu_weights`` and the
per-layer ``precompute`` driver, implemented in ``narhip.factor_pipeline``.
``compact_wy`` and ``RotationFactor`` come from there too; a
``RotationFactor`` loaded by the reference's own module works as well (the
fold reads only its fields).
"""

from __future__ import annotations

import argparse
from pathlib import Path

import torch

from narhip.factor_pipeline import (FoldedR4, RotationFactor, block_hadamard_columns,  # noqa: F401
                                    compact_wy, fold_swiglu_weights, signed_permute_rows, signs_for,
                                    source_for_target)


def precompute(workdir: Path, model: str, rank: int, layers: int, seed: int) -> None:
    """Fold every layer's calibrated factor and store the online factors (no dense R)."""
    device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    root = workdir / "activations" / model / "e11_calibration" / "factors" / f"nar_b128_k{rank}"
    output = workdir / "artifacts" / "e17v2" / model / f"k{rank}"
    for layer in range(layers):
        factor = RotationFactor.load(root / f"down_layer_{layer:02d}.pt", device)
        folded = FoldedR4.from_factor(factor, signs_for(factor.n, layer, seed, device))
        folded.save(output / f"down_layer_{layer:02d}.pt", {"model": model, "layer": layer})


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--workdir", type=Path, required=True)
    parser.add_argument("--model", required=True)
    parser.add_argument("--rank", type=int, choices=(8, 32), required=True)
    parser.add_argument("--layers", type=int, required=True)
    parser.add_argument("--seed", type=int, default=20260902)
    args = parser.parse_args()
    precompute(args.workdir.resolve(), args.model, args.rank, args.layers, args.seed)


if __name__ == "__main__":
    main()
