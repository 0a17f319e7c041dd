"""Portable seeded synthetic inputs: splitmix64 -> Box-Muller, in numpy.

Bit-for-bit the same on every platform and numpy version (integer mixing in
uint64, transcendental work in float64, one final cast to float32), so test
inputs and fixtures do not depend on a library's RNG implementation.
Seed convention for the benchmark configurations: 0x1F0000 + config*1000 +
index.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at `seed`."""
    with np.errstate(over="ignore"):
        state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = state
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """float32 N(0, std^2) samples of the given shape."""
    n = int(np.prod(shape))
    pairs = (n + 1) // 2
    z = splitmix64(seed, 2 * pairs)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53  # (0, 1]
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53          # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, dtype=np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (out[:n] * std).astype(np.float32).reshape(shape)


def uniform_ints(seed: int, n: int, high: int) -> np.ndarray:
    """n int32 values uniform in [0, high)."""
    z = splitmix64(seed, n)
    return (z % np.uint64(high)).astype(np.int32)


def config_seed(config: int, index: int) -> int:
    return 0x1F0000 + config * 1000 + index
