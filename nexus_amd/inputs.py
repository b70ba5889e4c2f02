"""Seeded synthetic inputs for the attention path (numpy, deterministic on any machine).

Values are N(0, 1) from splitmix64 -> Box-Muller; tensor t of a case uses seed + t
(Q: seed, K: seed + 1, V: seed + 2).  K/V are rounded to f16 either round-to-nearest-even
(numpy's cast) or with the KV cache's truncating store conversion (kvcache.h:903-911).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 started at `seed` (outputs 1..n of the sequence)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int) -> np.ndarray:
    """n N(0,1) float32 values (Box-Muller on pairs of 53-bit uniforms)."""
    z = splitmix64(seed, 2 * n)
    u = (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log1p(-u1))
    return (r * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def f32_to_f16_trunc(x: np.ndarray) -> np.ndarray:
    """The KV cache store conversion: truncate the mantissa, flush f16 subnormals to
    signed zero, overflow (and nan) to +-inf.  Returns uint16 bit patterns."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    sign = ((b >> 16) & 0x8000).astype(np.uint16)
    e16 = ((b >> 23) & 0xFF).astype(np.int32) - 112
    mant = ((b >> 13) & 0x3FF).astype(np.uint16)
    out = sign | (np.clip(e16, 0, 31).astype(np.uint16) << 10) | mant
    out = np.where(e16 <= 0, sign, out)
    out = np.where(e16 >= 31, sign | np.uint16(0x7C00), out)
    return out.astype(np.uint16)


def f16_bits(x: np.ndarray, mode: str = "rne") -> np.ndarray:
    if mode == "rne":
        return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
    if mode == "trunc":
        return f32_to_f16_trunc(x)
    raise ValueError(mode)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def make_case(*, n_q_heads: int, n_kv_heads: int, head_dim: int, n_query: int, n_ctx: int,
              kv_stride: int | None = None, seed: int = 1234, q_f16: bool = False,
              kv_round: str = "rne", q_scale: float = 1.0):
    """Q (f32 values, N(0, q_scale^2), f16-exact when q_f16), K/V f16 bits [Hkv][kv_stride][hd].
    Rows of K/V past n_ctx (stride padding) are filled with a large finite sentinel so a
    kernel that reads them produces visibly wrong results."""
    stride = n_ctx if kv_stride is None else kv_stride
    q = normal(seed, n_query * n_q_heads * head_dim).reshape(n_query, n_q_heads, head_dim)
    if q_scale != 1.0:
        q = (q * np.float32(q_scale)).astype(np.float32)
    if q_f16:
        q = q.astype(np.float16).astype(np.float32)
    k = np.full((n_kv_heads, stride, head_dim), 0x7BFF, dtype=np.uint16)   # 65504
    v = np.full((n_kv_heads, stride, head_dim), 0x7BFF, dtype=np.uint16)
    kn = normal(seed + 1, n_kv_heads * n_ctx * head_dim).reshape(n_kv_heads, n_ctx, head_dim)
    vn = normal(seed + 2, n_kv_heads * n_ctx * head_dim).reshape(n_kv_heads, n_ctx, head_dim)
    k[:, :n_ctx] = f16_bits(kn, kv_round)
    v[:, :n_ctx] = f16_bits(vn, kv_round)
    return q, k, v
