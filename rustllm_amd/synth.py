"""Seeded synthetic inputs: splitmix64 -> uniform [0, 1) -> Box-Muller.

N(mu, sigma) takes sigma as the standard deviation.  Seeds are derived from
a text key (op, dtype, shape) with CRC32 so every run and every host draws
the same values.
"""

from __future__ import annotations

import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def seed_for(*parts) -> int:
    """Stable 64-bit seed from the parts' text."""
    text = "|".join(str(p) for p in parts).encode()
    lo = zlib.crc32(text)
    hi = zlib.crc32(text[::-1] + b"#")
    return (hi << 32) | lo


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at `seed` (uint64)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """n doubles in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, shape, mu: float = 0.0, sigma: float = 1.0, dtype=np.float32):
    n = int(np.prod(shape, dtype=np.int64))
    u = uniform(seed, 2 * n)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mu + sigma * z).astype(dtype).reshape(shape)


def uniform_range(seed: int, shape, lo: float, hi: float, dtype=np.float32):
    n = int(np.prod(shape, dtype=np.int64))
    return (lo + (hi - lo) * uniform(seed, n)).astype(dtype).reshape(shape)
