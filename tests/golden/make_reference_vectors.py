"""Write golden vectors for the oracle from the reference's own functions.

Run in the build container only (the reference is never shipped):

    NAR_REFERENCE=/root/reference python tests/golden/make_reference_vectors.py

It imports the reference's pure-PyTorch functions for the parts of the path
that closed forms and invariants cannot pin on their own -- the exact +-1
pattern and orientation of the Paley factors, the Kronecker row layout of
full_hadamard_rows, the quantizer's degenerate-group handling, and the sign
convention of the rank-k row form -- and stores their inputs and outputs as
data in reference_vectors.npz.  The E0 known answers are copied from the
reference's results/e0.json into e0_reference.json.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path(os.environ.get("NAR_REFERENCE", "/root/reference"))
HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(REF))
sys.path.insert(0, str(REF / "quarot-llama3"))

from nar import activation_experiments as act  # noqa: E402
from nar import experiment as base  # noqa: E402
from nar import extended_experiment as ext  # noqa: E402


def f16bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main() -> None:
    rng = np.random.default_rng(20260902)
    out: dict[str, np.ndarray] = {}

    # Paley factors exactly as the reference builds them (fp32, normalised).
    out["paley12"] = ext._paley_hadamard_12(torch.device("cpu"), torch.float32).numpy()
    out["paley28"] = act.paley_hadamard_28(torch.device("cpu"), torch.float32).numpy()

    # full_hadamard_rows: Kronecker layout, orientation, dispatch order, signs.
    shapes = [(5, 112), (3, 224), (4, 48), (4, 192), (2, 3072), (2, 14336), (6, 128), (2, 1024)]
    for i, (t, n) in enumerate(shapes):
        x = (rng.standard_normal((t, n)) * rng.choice([0.1, 1.0, 30.0], size=(t, 1))).astype(np.float32)
        s = rng.choice(np.array([-1.0, 1.0], np.float32), size=n).astype(np.float32)
        y = act.full_hadamard_rows(torch.from_numpy(x), torch.from_numpy(s)).numpy()
        out[f"fhr{i}_x"], out[f"fhr{i}_s"], out[f"fhr{i}_y"] = x, s, y

    # Plain FWHT (stage order pinned) on power-of-two widths.
    for q in (32, 128, 512, 1024):
        x = rng.standard_normal((4, q)).astype(np.float32) * np.float32(3.0)
        x[0, ::7] *= np.float32(1e4)
        out[f"fwht{q}_x"] = x
        out[f"fwht{q}_y"] = ext._fast_walsh_hadamard(torch.from_numpy(x)).numpy()

    # dynamic_asym_int4 on the special-case suite and adversarial groups.
    n = 256
    base_row = rng.standard_normal(n).astype(np.float32)
    cases = {
        "zero": np.zeros((2, n), np.float32),
        "constant": np.full((2, n), 0.5, np.float32),
        "rounding_boundary": np.tile(((np.arange(n) % 15 - 7 + 0.5) / 7).astype(np.float32), (2, 1)),
        "common_offset": np.tile((64 + base_row * 0.03125).astype(np.float32), (2, 1)),
        "outlier": np.tile(base_row, (2, 1)),
        "random": rng.standard_normal((8, n)).astype(np.float32),
        "scaled": (rng.standard_normal((8, n)) * np.float32(1e3)).astype(np.float32),
        "tiny_range": (np.float32(0.5) + rng.standard_normal((4, n)).astype(np.float32) * np.float32(1e-7)).astype(np.float32),
        "subnormal_scale": (rng.standard_normal((4, n)) * np.float32(1e-6)).astype(np.float32),
        "huge": (rng.standard_normal((2, n)) * np.float32(1e5)).astype(np.float32),
    }
    cases["outlier"][:, 0] = 128.0
    fp16_hazard = np.full((1, n), 0.5, np.float32)
    fp16_hazard[0, 1] = np.float32(0.5 + 4e-7)
    cases["fp16_hazard"] = fp16_hazard
    near_const = rng.standard_normal((4, n)).astype(np.float32)
    near_const[:, :128] = near_const[:, :1] + (rng.standard_normal((4, 128)) * 1e-9).astype(np.float32)
    cases["near_constant"] = near_const
    names = []
    for name, x in cases.items():
        for b in (32, 64, 128):
            deq, s16, z16, codes = base.dynamic_asym_int4(torch.from_numpy(x), b)
            key = f"q_{name}_b{b}"
            out[key + "_x"] = x
            out[key + "_deq"] = deq.numpy()
            out[key + "_scale"] = f16bits(s16)
            out[key + "_zero"] = f16bits(z16)
            out[key + "_codes"] = codes.reshape(x.shape[0], -1).numpy()
            names.append(key)
    out["q_names"] = np.array(names)

    # Rank-k row form with the block-H128 factor: H x - (x Y') W''^T.
    try:
        import nar_r4_kernel as nk  # imports triton; only the pure-torch function is called
        have_nk = True
    except Exception as error:  # noqa: BLE001
        print("nar_r4_kernel import failed:", error)
        have_nk = False
    for i, (t, n, k) in enumerate([(4, 256, 8), (3, 384, 2)]):
        x = rng.standard_normal((t, n)).astype(np.float32)
        y = (rng.standard_normal((n, k)) / np.sqrt(n)).astype(np.float32)
        w = (rng.standard_normal((k, n)) / np.sqrt(n)).astype(np.float32)
        out[f"rt{i}_x"], out[f"rt{i}_y"], out[f"rt{i}_w"] = x, y, w
        if have_nk:
            out[f"rt{i}_out"] = nk.reference_transform(torch.from_numpy(x), torch.from_numpy(y),
                                                       torch.from_numpy(w)).numpy()

    np.savez_compressed(HERE / "reference_vectors.npz", **out)

    e0 = json.loads((REF / "results" / "e0.json").read_text())
    (HERE / "e0_reference.json").write_text(json.dumps(
        {"source": "results/e0.json", "seed": e0["seed"], "rows": e0["rows"]}, indent=1) + "\n")
    print("wrote", HERE / "reference_vectors.npz", sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main()
