"""Seeded synthetic KV / query data, bit-identical on any host.

A counter-based generator (splitmix64 over ``seed * 2**32 + index``, then
Box-Muller) written with numpy integer ops only, so the GPU box regenerates the
exact inputs the committed fixtures were made from without depending on the
torch or numpy RNG version.

The benchmark configs add "outlier channels": a fixed number of head_dim
channels per KV head, chosen by the seed, multiplied by a factor in fp32
before the single cast to fp16.
"""
from __future__ import annotations

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = (x + np.uint64(0x9E3779B97F4A7C15)) & _M64
    z = x
    z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & _M64
    z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & _M64
    return z ^ (z >> np.uint64(31))


def uniform01(n: int, seed: int, offset: int = 0) -> np.ndarray:
    """n float64 values in (0, 1) from stream ``seed``."""
    idx = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        base = np.uint64((seed & 0xFFFFFFFF) << 32)
        r = _splitmix64(idx + base)
    return ((r >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """float32 N(0, std^2) of ``shape`` (Box-Muller, both outputs used)."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u1 = uniform01(m, seed, 0)
    u2 = uniform01(m, seed, m)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * std).astype(np.float32).reshape(shape)


def outlier_channels(n_heads: int, head_dim: int, n_out: int, seed: int) -> np.ndarray:
    """[n_heads, n_out] distinct channel indices per head (seeded)."""
    out = np.empty((n_heads, n_out), dtype=np.int64)
    u = uniform01(n_heads * head_dim, seed ^ 0x5A5A5A5A)
    for h in range(n_heads):
        order = np.argsort(u[h * head_dim:(h + 1) * head_dim], kind="stable")
        out[h] = np.sort(order[:n_out])
    return out


def kv_tensor(B: int, H: int, T: int, D: int, seed: int, n_out: int = 0, factor: float = 1.0,
              std: float = 1.0) -> np.ndarray:
    """fp16 [B,H,T,D] N(0,std) with ``n_out`` outlier channels per head scaled by ``factor``."""
    x = normal((B, H, T, D), seed, std)
    if n_out:
        ch = outlier_channels(H, D, n_out, seed)
        for h in range(H):
            x[:, h, :, ch[h]] *= np.float32(factor)
    return x.astype(np.float16)
