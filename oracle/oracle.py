"""Python face of the CPU oracle for the NAR rotate-and-quantize path.

TEST INFRASTRUCTURE ONLY: the restatement the HIP kernels are tested against.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product package (nar-offline-validation_amd/) never does.

The arithmetic lives in nar_oracle.c (see its header for the reference
file:line each step follows).  This module adds numpy conversions, the
tie-aware comparators used by the parity tests, and the quantization metrics
of nar/experiment.py:186-199.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libnar_oracle.so"

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from . import build as _build  # type: ignore
            _build.build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        _lib.nar_oracle_rotate.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
            f32p, ctypes.c_int64]
        _lib.nar_oracle_rotate.restype = ctypes.c_int
        _lib.nar_oracle_projection.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int64,
            f32p, f32p]
        _lib.nar_oracle_projection.restype = ctypes.c_int
        _lib.nar_oracle_quant.argtypes = [
            f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib.nar_oracle_quant.restype = ctypes.c_int
        _lib.nar_oracle_paley.argtypes = [ctypes.c_int, ctypes.c_void_p]
        _lib.nar_oracle_paley.restype = ctypes.c_int
        _lib.nar_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.nar_oracle_f32_to_f16.restype = ctypes.c_uint16
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------ conversions ---

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even (torch `.to(bfloat16)`)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.ascontiguousarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# -------------------------------------------------------------- operators ---

def paley(m: int) -> np.ndarray:
    out = np.zeros((m, m), dtype=np.int8)
    if lib().nar_oracle_paley(m, _ptr(out)) != 0:
        raise ValueError(f"no Paley construction for order {m}")
    return out


def rotate(x: np.ndarray, m: int, q: int, signs: np.ndarray | None = None,
           v: np.ndarray | None = None, wt: np.ndarray | None = None,
           rank_block: int | None = None) -> np.ndarray:
    """x' = H_s x - (x V) W^T on fp32 rows [T, n] (exact fp32 input)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, n = x.shape
    k = 0 if v is None else int(v.shape[1])
    nb = n if rank_block is None else int(rank_block)
    out = np.empty((T, n), dtype=np.float32)
    s = None if signs is None else np.ascontiguousarray(signs, dtype=np.float32)
    vv = None if v is None else np.ascontiguousarray(v, dtype=np.float32)
    ww = None if wt is None else np.ascontiguousarray(wt, dtype=np.float32)
    rc = lib().nar_oracle_rotate(x, T, n, n, m, q, _ptr(s), k, nb, _ptr(vv), _ptr(ww), out, n)
    if rc != 0:
        raise ValueError(f"oracle rotate rejected shape n={n} m={m} q={q} k={k} nb={nb}")
    return out


def projection(x: np.ndarray, v: np.ndarray, rank_block: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, n = x.shape
    k = int(v.shape[1])
    nb = n if rank_block is None else int(rank_block)
    u = np.empty((T, (n // nb) * k), dtype=np.float32)
    if lib().nar_oracle_projection(x, T, n, n, k, nb, np.ascontiguousarray(v, np.float32), u) != 0:
        raise ValueError("oracle projection rejected shape")
    return u


@dataclass
class Quantized:
    codes: np.ndarray      # uint8 [T, n], one code per channel
    packed: np.ndarray     # uint8 [T, n/2]
    scales: np.ndarray     # uint16 fp16 bits [T, n/b]
    zeros: np.ndarray      # uint16 fp16 bits [T, n/b]
    deq: np.ndarray        # fp32 [T, n]


def quant(xr: np.ndarray, b: int) -> Quantized:
    xr = np.ascontiguousarray(xr, dtype=np.float32)
    T, n = xr.shape
    codes = np.empty((T, n), np.uint8)
    packed = np.empty((T, n // 2), np.uint8)
    scales = np.empty((T, n // b), np.uint16)
    zeros = np.empty((T, n // b), np.uint16)
    deq = np.empty((T, n), np.float32)
    if lib().nar_oracle_quant(xr, T, n, n, b, _ptr(codes), _ptr(packed), _ptr(scales),
                              _ptr(zeros), _ptr(deq)) != 0:
        raise ValueError("oracle quant rejected shape")
    return Quantized(codes, packed, scales, zeros, deq)


def unpack(packed: np.ndarray, n: int) -> np.ndarray:
    """Low nibble = even channel (nar/kernels/r4_fused_v2.py:358-361)."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (n,), np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = packed >> 4
    return out


def dequant(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, n: int, b: int) -> np.ndarray:
    q = unpack(packed, n).reshape(packed.shape[0], n // b, b).astype(np.float32)
    s = f16_bits_to_f32(scales)[..., None]
    z = f16_bits_to_f32(zeros)[..., None]
    return ((q * s).astype(np.float32) + z).astype(np.float32).reshape(packed.shape[0], n)


def nmse(x: np.ndarray, deq: np.ndarray) -> float:
    """sum (deq - x)^2 / sum x^2 with fp64 sums (nar/experiment.py:192-199)."""
    x64 = x.astype(np.float64)
    return float(((deq.astype(np.float64) - x64) ** 2).sum() / max((x64 ** 2).sum(), np.finfo(np.float64).tiny))


# ------------------------------------------------------------ comparators ---

def _f16_neighbour_midpoints(bits_a: np.ndarray, bits_b: np.ndarray) -> np.ndarray:
    a = f16_bits_to_f32(bits_a).astype(np.float64)
    b = f16_bits_to_f32(bits_b).astype(np.float64)
    return 0.5 * (a + b)


@dataclass
class ParityReport:
    elements: int
    groups: int
    code_mismatch: int
    code_mismatch_unexplained: int
    code_max_abs_diff: int
    scale_mismatch: int
    scale_mismatch_unexplained: int
    zero_mismatch: int
    zero_mismatch_unexplained: int

    @property
    def code_mismatch_fraction(self) -> float:
        return self.code_mismatch / max(1, self.elements)

    @property
    def meta_mismatch_fraction(self) -> float:
        return (self.scale_mismatch + self.zero_mismatch) / max(1, 2 * self.groups)

    def exact(self) -> bool:
        return self.code_mismatch == 0 and self.scale_mismatch == 0 and self.zero_mismatch == 0

    def within_contract(self, max_fraction: float = 1e-4) -> bool:
        """Codes +-1 and scale/zero 1-ulp only at rounding ties, on <= max_fraction."""
        return (self.code_max_abs_diff <= 1
                and self.code_mismatch_unexplained == 0
                and self.scale_mismatch_unexplained == 0
                and self.zero_mismatch_unexplained == 0
                and self.code_mismatch_fraction <= max_fraction
                and self.meta_mismatch_fraction <= max_fraction)


def compare_quant(ref_rot: np.ndarray, ref: Quantized, codes_obs: np.ndarray,
                  scales_obs: np.ndarray, zeros_obs: np.ndarray, b: int,
                  rel_err: float = 0.0) -> ParityReport:
    """Classify every difference between observed and oracle INT4 outputs.

    rel_err is the documented bound on the observed path's rotated values,
    |x'_obs - x'_oracle| <= rel_err * (|x'| + rms(row)).  A difference counts as
    a rounding tie (explained) only where the oracle's pre-rounding value lies
    within that bound of the rounding boundary it straddles:
      * scale : raw (hi-lo)/15 within the bound of the fp16 midpoint
      * zero  : lo within the bound of the fp16 midpoint
      * code  : |(x'-z)/s - (k+1/2)| within the bound, or the group's scale or
                zero differs (a tie there moves every code of the group).
    With rel_err = 0 nothing is explained and any difference fails.
    """
    T, n = ref_rot.shape
    G = n // b
    xr = ref_rot.astype(np.float64).reshape(T, G, b)
    row_rms = np.sqrt((ref_rot.astype(np.float64) ** 2).mean(axis=1)).reshape(T, 1, 1)
    err = rel_err * (np.abs(xr) + row_rms)                          # per element bound
    lo = xr.min(axis=2)
    hi = xr.max(axis=2)
    lo_err = err.max(axis=2)
    s_ref = f16_bits_to_f32(ref.scales).astype(np.float64)
    z_ref = f16_bits_to_f32(ref.zeros).astype(np.float64)

    scale_diff = scales_obs != ref.scales
    zero_diff = zeros_obs != ref.zeros
    one_ulp_s = np.abs(scales_obs.astype(np.int32) - ref.scales.astype(np.int32)) == 1
    one_ulp_z = np.abs(zeros_obs.astype(np.int32) - ref.zeros.astype(np.int32)) == 1
    raw = (hi - lo) / 15.0
    mid_s = _f16_neighbour_midpoints(scales_obs, ref.scales)
    mid_z = _f16_neighbour_midpoints(zeros_obs, ref.zeros)
    s_tie = np.abs(raw - mid_s) <= (2 * lo_err / 15.0 + 2.0 ** -22 * np.abs(raw))
    z_tie = np.abs(lo - mid_z) <= (lo_err + 2.0 ** -23 * np.abs(lo))
    scale_unexplained = scale_diff & ~(one_ulp_s & s_tie & (rel_err > 0))
    zero_unexplained = zero_diff & ~(one_ulp_z & z_tie & (rel_err > 0))

    co = codes_obs.reshape(T, G, b).astype(np.int32)
    cr = ref.codes.reshape(T, G, b).astype(np.int32)
    cdiff = co != cr
    quot = (xr - z_ref[..., None]) / s_ref[..., None]
    frac_dist = np.abs(quot - np.floor(quot) - 0.5)
    q_err = (err + np.abs(z_ref[..., None]) * rel_err) / s_ref[..., None] + 1e-6
    code_tie = frac_dist <= q_err
    meta = (scale_diff | zero_diff)[..., None]
    code_unexplained = cdiff & ~((code_tie | meta) & (rel_err > 0))
    return ParityReport(
        elements=T * n, groups=T * G,
        code_mismatch=int(cdiff.sum()),
        code_mismatch_unexplained=int(code_unexplained.sum()),
        code_max_abs_diff=int(np.abs(co - cr).max()) if co.size else 0,
        scale_mismatch=int(scale_diff.sum()),
        scale_mismatch_unexplained=int(scale_unexplained.sum()),
        zero_mismatch=int(zero_diff.sum()),
        zero_mismatch_unexplained=int(zero_unexplained.sum()),
    )


def rotated_error(obs: np.ndarray, ref: np.ndarray) -> float:
    """max |obs - ref| / (|ref| + rms(row)) -- the quantity rel_err bounds."""
    ref64 = ref.astype(np.float64)
    rms = np.sqrt((ref64 ** 2).mean(axis=1, keepdims=True))
    return float((np.abs(obs.astype(np.float64) - ref64) / (np.abs(ref64) + rms + 1e-300)).max())


def relative_l2(obs: np.ndarray, ref: np.ndarray) -> float:
    ref64 = ref.astype(np.float64)
    return float(np.linalg.norm(obs.astype(np.float64) - ref64) / max(np.linalg.norm(ref64), 1e-30))


def sqrt_f32(q: int) -> np.float32:
    return np.float32(math.sqrt(q))


def w4a4_gemm(a_packed: np.ndarray, a_s: np.ndarray, a_z: np.ndarray, w_packed: np.ndarray,
              w_s: np.ndarray, w_z: np.ndarray, n: int, b: int = 128) -> np.ndarray:
    """fp64 [T, O] = dequant(A) dequant(W)^T: each operand dequantized as the
    reference's dequantize does (fp32 q * s, then + z; nar/kernels/r4_fused_v2.py:
    364-369), the products summed exactly in fp64.  The group-asymmetric GEMM the
    packed format feeds (quarot-llama3/e28_v2/docs/quantizer_contract.md:134-140)."""
    da = dequant(a_packed, a_s, a_z, n, b).astype(np.float64)
    dw = dequant(w_packed, w_s, w_z, n, b).astype(np.float64)
    return da @ dw.T


def w4a4_group_formula(a_packed: np.ndarray, a_s: np.ndarray, a_z: np.ndarray, w_packed: np.ndarray,
                       w_s: np.ndarray, w_z: np.ndarray, n: int, b: int = 128) -> np.ndarray:
    """The same product from the per-group four-term form, exact in fp64:
    sum_g sA sW sum qA qW + sA zW sum qA + zA sW sum qW + b zA zW."""
    qa = unpack(a_packed, n).astype(np.int64).reshape(a_packed.shape[0], n // b, b)
    qw = unpack(w_packed, n).astype(np.int64).reshape(w_packed.shape[0], n // b, b)
    sa, za = f16_bits_to_f32(a_s).astype(np.float64), f16_bits_to_f32(a_z).astype(np.float64)
    sw, zw = f16_bits_to_f32(w_s).astype(np.float64), f16_bits_to_f32(w_z).astype(np.float64)
    dot = np.einsum("tgj,ogj->tog", qa, qw).astype(np.float64)
    sum_a, sum_w = qa.sum(-1).astype(np.float64), qw.sum(-1).astype(np.float64)
    y = (np.einsum("tg,og,tog->to", sa, sw, dot) + np.einsum("tg,og,tg->to", sa, zw, sum_a)
         + np.einsum("tg,og,og->to", za, sw, sum_w) + b * np.einsum("tg,og->to", za, zw))
    return y
