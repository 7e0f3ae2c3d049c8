"""Write golden vectors for the quantizer on groups holding NaN or +-Inf.

Run in the build container only (the reference is never shipped):

    NAR_REFERENCE=/root/reference python tests/golden/make_nonfinite_vectors.py

dynamic_asym_int4 (nar/experiment.py:158-184) reduces each group with
torch.amin / torch.amax, which propagate NaN, so a group holding a NaN gets
scale 1, a NaN zero-point and NaN dequantized values; an Inf widens the range
to Inf.  The inputs and the reference's outputs are stored as data in
nonfinite_vectors.npz.
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

from nar import experiment as base  # noqa: E402

NEG_NAN = np.array([0xFFC00000], np.uint32).view(np.float32)[0]


def f16bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def cases(rng: np.random.Generator, n: int) -> dict[str, np.ndarray]:
    def rows(r=4):
        return rng.standard_normal((r, n)).astype(np.float32)
    out = {}
    x = rows(); x[0, 5] = np.nan; x[1, 100] = np.nan; x[2, 200] = np.nan; x[3, 33] = np.nan
    out["nan_one"] = x
    x = rows(); x[0, :32] = np.nan; x[1, 128:256] = np.nan; x[2, 64:96] = np.nan; x[3, :] = np.nan
    out["nan_all"] = x
    x = rows(); x[0, 7] = NEG_NAN; x[1, 130] = NEG_NAN; x[2, 255] = NEG_NAN
    out["neg_nan"] = x
    x = rows(); x[0, 3] = np.inf; x[1, 129] = np.inf; x[2, 250] = np.inf; x[3, 64] = np.inf
    out["pos_inf"] = x
    x = rows(); x[0, 3] = -np.inf; x[1, 129] = -np.inf; x[2, 250] = -np.inf; x[3, 64] = -np.inf
    out["neg_inf"] = x
    x = rows(); x[:, 10] = np.inf; x[:, 20] = -np.inf; x[:, 140] = np.inf; x[:, 141] = -np.inf
    out["both_inf"] = x
    x = rows(); x[0, :32] = np.inf; x[1, :128] = -np.inf; x[2, 128:] = np.inf; x[3, 32:64] = -np.inf
    out["all_inf"] = x
    x = rows(); x[:, 2] = np.inf; x[:, 3] = np.nan; x[:, 130] = -np.inf; x[:, 200] = np.nan
    out["inf_nan"] = x
    x = rows(); x[:, 1] = np.float32(3e38); x[:, 2] = np.float32(-3e38); x[:, 160] = np.float32(3.4e38)
    out["huge_range"] = x
    return out


def main() -> None:
    rng = np.random.default_rng(20261202)
    n = 256
    out: dict[str, np.ndarray] = {}
    names = []
    with np.errstate(invalid="ignore"):
        for name, x in cases(rng, n).items():
            for b in (32, 64, 128):
                deq, s16, z16, codes = base.dynamic_asym_int4(torch.from_numpy(x), b)
                key = f"nf_{name}_b{b}"
                out[key + "_x"] = x
                out[key + "_deq"] = deq.numpy()
                out[key + "_scale"] = f16bits(s16)
                out[key + "_zero"] = f16bits(z16)
                out[key + "_codes"] = codes.reshape(x.shape[0], -1).numpy()
                names.append(key)
    out["nf_names"] = np.array(names)
    np.savez_compressed(HERE / "nonfinite_vectors.npz", **out)
    print("wrote", HERE / "nonfinite_vectors.npz", len(names), "cases")


if __name__ == "__main__":
    main()
