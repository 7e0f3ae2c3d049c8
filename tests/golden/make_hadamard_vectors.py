"""Write golden vectors for the Hadamard widths added to the hooks' domain.

Run in the build container only (the reference is never shipped):

    NAR_REFERENCE=/root/reference python tests/golden/make_hadamard_vectors.py

It imports the reference's pure-PyTorch full_hadamard_rows and paley_hadamard
for what closed forms alone cannot pin -- the +-1 pattern and orientation of
the Qwen3 Paley factors (orders 20, 68, 76, 200), the dispatch of
full_hadamard_rows to them, and its power-of-two branch beyond 1024 channels
-- and stores their inputs and outputs as data in hadamard_vectors.npz.
Inputs are bf16-representable fp32 values (what the GPU kernels read).
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


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def main() -> None:
    rng = np.random.default_rng(20261202)
    out: dict[str, np.ndarray] = {}
    cpu = torch.device("cpu")
    for order in (20, 68, 76, 200):
        h = act.paley_hadamard(order, cpu, torch.float64).numpy()
        out[f"paley{order}_sign"] = np.sign(h).astype(np.int8)
        out[f"paley{order}_scale"] = np.array([np.abs(h).max()], dtype=np.float64)
    shapes = [(3, 2048), (2, 4096), (2, 8192), (3, 2560), (2, 5120), (1, 9728), (1, 17408)]
    for i, (t, n) in enumerate(shapes):
        x = rng.standard_normal((t, n)) * rng.choice([0.05, 1.0, 40.0], size=(t, 1))
        x[:, rng.choice(n, size=4, replace=False)] *= 30.0
        x = bf16_round(x.astype(np.float32))
        s = rng.choice(np.array([-1.0, 1.0], np.float32), size=n).astype(np.float32)
        y = act.full_hadamard_rows(torch.from_numpy(x), torch.from_numpy(s)).numpy()
        out[f"fhr{i}_x"], out[f"fhr{i}_s"], out[f"fhr{i}_y"] = x, s, y
    np.savez_compressed(HERE / "hadamard_vectors.npz", **out)
    print(f"wrote {HERE / 'hadamard_vectors.npz'}: {sorted(out)}")


if __name__ == "__main__":
    main()
