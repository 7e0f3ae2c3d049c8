"""Seeded synthetic inputs for the five benchmark shapes of the path.

Each generator is deterministic (numpy PCG64, one generator per component, so
the first t rows of a shape do not depend on how many rows were asked for) and
returns host arrays:

  x       bf16 bit patterns, uint16 [T, n] (fp32 values rounded to nearest even)
  v       fp32 [n, k]   projection factor Y'
  w_t     fp32 [k, n]   correction factor W''^T = -U^T, so x' = H x + U (V^T x)

Shapes (tokens x channels, Hadamard, rank, group):
  kcache_3b     2048 x (8 heads x 128), H_128 per head, k=2 per head, b=32
  qproj_3b      4096 x 3072,  H_12 (x) H_256,  k=16, b=64
  downproj_8b   8192 x 14336, H_28 (x) H_512,  k=32, b=128
  vcache_decode 64 x (8 heads x 128), H_128 per head, k=4 per head, b=32,
                codes scattered into a 64 x 4096-slot packed cache
  downproj_70b  16384 x 28672, H_28 (x) H_1024, k=64, b=128
plus the reference's E17 fused-kernel settings (block H_128, T=2048, k=8/32)
for comparison with its published timings.
The base seed is the reference's DEFAULT_SEED (nar/experiment.py:38).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

BASE_SEED = 20260902


def _rng(config: int, component: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(BASE_SEED + 1000 * config + component))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def orthonormal(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    q, r = np.linalg.qr(rng.standard_normal((n, k)))
    return (q * np.sign(np.diag(r))).astype(np.float32)


@dataclass
class Workload:
    name: str
    x: np.ndarray                  # uint16 bf16 bits [T, n]
    hadamard: tuple[int, int]
    group: int
    v: np.ndarray | None = None    # fp32 [n, k]
    w_t: np.ndarray | None = None  # fp32 [k, n]
    rank_block: int | None = None
    dest_rows: np.ndarray | None = None
    out_rows: int | None = None
    meta: dict = field(default_factory=dict)

    @property
    def tokens(self) -> int:
        return int(self.x.shape[0])

    @property
    def n(self) -> int:
        return int(self.x.shape[1])

    @property
    def k(self) -> int:
        return 0 if self.v is None else int(self.v.shape[1])

    @property
    def transform_f16(self) -> bool:
        """E28's fp16-in / fp16-out transform (x holds fp16 bits, no quantizer)."""
        return self.meta.get("io") == "f16"

    def algorithmic_bytes(self) -> int:
        """T*(2n + n/2 + 4n/b) + factor bytes read once (fp32 U, V); fp16 transform: T*4n + factors."""
        t, n, b = self.tokens, self.n, self.group
        factors = 0 if self.v is None else self.v.nbytes + self.w_t.nbytes
        if self.transform_f16:
            return t * 4 * n + factors
        return t * (2 * n + n // 2 + 4 * n // b) + factors


def _per_head_factors(rng: np.random.Generator, heads: int, d: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    vs, us = [], []
    for _ in range(heads):
        vs.append(orthonormal(rng, d, k))
        us.append(orthonormal(rng, d, k))
    v = np.concatenate(vs, axis=0)
    w_t = -np.concatenate(us, axis=0).T
    return np.ascontiguousarray(v), np.ascontiguousarray(w_t, dtype=np.float32)


def kcache_3b(tokens: int = 2048) -> Workload:
    """Post-RoPE K, 8 KV heads x 128: N(0,1), 4 outlier channels/head x20, RoPE theta=5e5."""
    heads, d, theta = 8, 128, 500000.0
    k_raw = _rng(1, 0).standard_normal((tokens, heads, d), dtype=np.float32)
    out_rng = _rng(1, 1)
    for h in range(heads):
        ch = out_rng.choice(d, size=4, replace=False)
        k_raw[:, h, ch] *= np.float32(20.0)
    inv_freq = theta ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(tokens, dtype=np.float64)[:, None] * inv_freq[None, :]
    emb = np.concatenate([ang, ang], axis=1)
    cos = np.cos(emb).astype(np.float32)[:, None, :]
    sin = np.sin(emb).astype(np.float32)[:, None, :]
    half = d // 2
    rot_half = np.concatenate([-k_raw[..., half:], k_raw[..., :half]], axis=-1)
    k_rope = (k_raw * cos + rot_half * sin).astype(np.float32)
    v, w_t = _per_head_factors(_rng(1, 2), heads, d, 2)
    return Workload("kcache_3b", bf16_bits(k_rope.reshape(tokens, heads * d)), (1, 128), 32,
                    v=v, w_t=w_t, rank_block=d, meta={"heads": heads, "head_dim": d})


def qproj_3b(tokens: int = 4096, full_tokens: int = 4096) -> Workload:
    """Student-t(4) activations + rank-8 spike (sigma 50..10) + 6 massive channels x100."""
    n = 3072
    x = _rng(2, 0).standard_t(4.0, size=(tokens, n)).astype(np.float32)
    srng = _rng(2, 1)
    a = orthonormal(srng, full_tokens, 8)[:tokens]
    b = orthonormal(srng, n, 8)
    sigma = np.linspace(50.0, 10.0, 8).astype(np.float32)
    x += (a * sigma[None, :]) @ b.T
    ch = _rng(2, 2).choice(n, size=6, replace=False)
    x[:, ch] *= np.float32(100.0)
    frng = _rng(2, 3)
    v = orthonormal(frng, n, 16)
    w_t = np.ascontiguousarray(-orthonormal(frng, n, 16).T)
    return Workload("qproj_3b", bf16_bits(x), (12, 256), 64, v=v, w_t=w_t)


def _silu_up(config: int, tokens: int, n: int, outliers: int) -> np.ndarray:
    g = _rng(config, 0).standard_normal((tokens, n), dtype=np.float32)
    u = _rng(config, 1).standard_normal((tokens, n), dtype=np.float32)
    x = g / (np.float32(1.0) + np.exp(-g)) * u
    ch = _rng(config, 2).choice(n, size=outliers, replace=False)
    x[:, ch] *= np.float32(50.0)
    return x


def downproj_8b(tokens: int = 8192) -> Workload:
    """SiLU(gate)*up, 16 outlier channels x50, H_28 (x) H_512, k=32, b=128."""
    n = 14336
    x = _silu_up(3, tokens, n, 16)
    frng = _rng(3, 3)
    v = orthonormal(frng, n, 32)
    w_t = np.ascontiguousarray(-orthonormal(frng, n, 32).T)
    return Workload("downproj_8b", bf16_bits(x), (28, 512), 128, v=v, w_t=w_t)


def vcache_decode_8b(batch: int = 64, slots: int = 4096) -> Workload:
    """One new V token per sequence, N(0, 0.5^2), scattered into seeded cache slots."""
    heads, d = 8, 128
    x = (_rng(4, 0).standard_normal((batch, heads * d), dtype=np.float32) * np.float32(0.5))
    v, w_t = _per_head_factors(_rng(4, 2), heads, d, 4)
    slot = _rng(4, 1).integers(0, slots, size=batch)
    dest = (np.arange(batch, dtype=np.int64) * slots + slot).astype(np.int64)
    return Workload("vcache_decode_8b", bf16_bits(x), (1, 128), 32, v=v, w_t=w_t, rank_block=d,
                    dest_rows=dest, out_rows=batch * slots, meta={"heads": heads, "slots": slots})


def downproj_70b(tokens: int = 16384) -> Workload:
    """SiLU(gate)*up, 32 outlier channels x50, H_28 (x) H_1024, k=64, b=128."""
    n = 28672
    x = _silu_up(5, tokens, n, 32)
    frng = _rng(5, 3)
    v = orthonormal(frng, n, 64)
    w_t = np.ascontiguousarray(-orthonormal(frng, n, 64).T)
    return Workload("downproj_70b", bf16_bits(x), (28, 1024), 128, v=v, w_t=w_t)


def _e17(config: int, tokens: int, n: int, k: int, outliers: int) -> np.ndarray:
    x = _silu_up(config, tokens, n, outliers)
    frng = _rng(config, 3)
    v = orthonormal(frng, n, k)
    w_t = np.ascontiguousarray(-orthonormal(frng, n, k).T)
    return x, v, w_t


def e17_8b(tokens: int = 2048, k: int = 8) -> Workload:
    """The reference's E17 fused-kernel setting (nar/e17_v3.py): Llama-3.1-8B down_proj
    input, 2048 tokens x 14336, block H_128, full-row rank k, b=128.  SiLU(gate)*up
    activations with 16 outlier channels x50 and orthonormal synthetic factors."""
    x, v, w_t = _e17(6 + (k == 32), tokens, 14336, k, 16)
    return Workload(f"e17_8b_k{k}", bf16_bits(x), (1, 128), 128, v=v, w_t=w_t)


def e17_3b(tokens: int = 2048, k: int = 8) -> Workload:
    """E17 on the Llama-3.2-3B down_proj width: 2048 tokens x 8192, block H_128, rank k, b=128."""
    x, v, w_t = _e17(8 + (k == 32), tokens, 8192, k, 16)
    return Workload(f"e17_3b_k{k}", bf16_bits(x), (1, 128), 128, v=v, w_t=w_t)


def e28(model: str = "8b", tokens: int = 2048, k: int = 8) -> Workload:
    """E28's down_proj transform (quarot-llama3/nar_r4_kernel.py NARDownTransform): fp16
    rows of the Llama-3.1-8B (14336) or Llama-3.2-3B (8192) down_proj input, H_128
    blocks, full-row rank k=8, fp16 out.  SiLU(gate)*up rows with 16 outliers x50."""
    n = {"8b": 14336, "3b": 8192}[model]
    x, v, w_t = _e17(10 + (model == "3b"), tokens, n, k, 16)
    bits = np.asarray(x, dtype=np.float16).view(np.uint16)
    return Workload(f"e28_{model}_T{tokens}", bits, (1, 128), 128, v=v, w_t=w_t, meta={"io": "f16"})


CONFIGS = {
    "kcache_3b": kcache_3b,
    "qproj_3b": qproj_3b,
    "downproj_8b": downproj_8b,
    "vcache_decode_8b": vcache_decode_8b,
    "downproj_70b": downproj_70b,
}

# The reference's published fused-kernel settings (block H_128), for comparison only.
REFERENCE_SETTINGS = {
    "e17_8b_k8": lambda: e17_8b(k=8),
    "e17_8b_k32": lambda: e17_8b(k=32),
    "e17_3b_k8": lambda: e17_3b(k=8),
    "e17_3b_k32": lambda: e17_3b(k=32),
    "e28_8b": lambda tokens=2048: e28("8b", tokens),
    "e28_3b": lambda tokens=2048: e28("3b", tokens),
}
