"""Write golden vectors for the offline factor pipeline from the reference's own functions.

Run in the build container only (the reference is never shipped):

    NAR_REFERENCE=/root/reference python tests/golden/make_factor_vectors.py

A small synthetic calibrated factor (n = 256, b = 128, six reflectors of which
one is inactive, random source/target orders) goes through the reference's
compact_wy (nar/e12_wy.py:46-66), FoldedR4.from_factor
(nar/fold_signed_permutation.py:70-120), FoldedR4.apply / q_unfolded and
RotationFactor.apply (nar/activation_experiments.py:292-299); inputs and
outputs are stored as data in factor_vectors.npz.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path(os.environ.get("NAR_REFERENCE", "/root/reference"))
HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(REF))

from nar import activation_experiments as act  # noqa: E402
from nar.e12_wy import compact_wy  # noqa: E402
from nar.fold_signed_permutation import FoldedR4  # noqa: E402


def main() -> None:
    g = torch.Generator().manual_seed(20260902)
    n, b, r = 256, 128, 6
    refl = torch.randn((r, n), generator=g)
    refl = refl / refl.norm(dim=1, keepdim=True)
    active = torch.tensor([True, True, False, True, True, True])
    source = torch.randperm(n, generator=g)
    target = torch.randperm(n, generator=g)
    signs = (torch.randint(0, 2, (n,), generator=g).float() * 2 - 1)
    x = torch.randn((5, n), generator=g) * 3.0
    factor = act.RotationFactor(n=n, b=b, reflectors=refl, active=active, source_order=source,
                                target_order=target, anchor_error=0.125)
    w, y = compact_wy(refl, active)
    folded = FoldedR4.from_factor(factor, signs)
    out = {
        "reflectors": refl.numpy(), "active": active.numpy(), "source_order": source.numpy(),
        "target_order": target.numpy(), "signs": signs.numpy(), "x": x.numpy(),
        "wy_w": w.numpy(), "wy_y": y.numpy(),
        "source_for_target": folded.source.numpy(),
        "y_prime_fp32": folded.y_prime_fp32.numpy(), "w_h_fp32": folded.w_h_fp32.numpy(),
        "w_h_t_fp32": folded.w_h_t_fp32.numpy(),
        "terms_bf16_bits": folded.y_prime_pad_terms_bf16.view(torch.int16).numpy(),
        "rotation_apply": factor.apply(x, signs).numpy(),
        "q_unfolded": folded.q_unfolded(x).numpy(),
        "folded_apply": folded.apply(folded.q_unfolded(x)).numpy(),
    }
    np.savez_compressed(HERE / "factor_vectors.npz", **out)
    print("wrote", HERE / "factor_vectors.npz", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
