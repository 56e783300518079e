"""Portable seeded inputs for the golden fixtures.

splitmix64 with the constants of the reference's yrng (platform.c:411-417),
computed with numpy uint64 arithmetic (exact and platform independent).
Value i of a stream uses generator state seed + (i+1)*GOLDEN; uniforms take
the top 24 bits like the reference (engine.c:1637, convert.c:164).
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def splitmix(seed: int, n: int, first: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        idx = np.arange(first + 1, first + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform_pm1(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    """float32 values (2u-1)*scale, u = (r>>40 + 0.5)/2^24 in (0,1)."""
    r = splitmix(seed, n)
    u = ((r >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0
    return ((2.0 * u - 1.0) * scale).astype(np.float32)
