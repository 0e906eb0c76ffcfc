"""The repository's one documented PRNG for synthetic inputs.

SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
generators", OOPSLA 2014): output i (i = 1, 2, ...) of a stream seeded with s
is mix(s + i * 0x9E3779B97F4A7C15) where
    mix(z): z ^= z >> 30; z *= 0xBF58476D1CE4E5B9;
            z ^= z >> 27; z *= 0x94D049BB133111EB; z ^= z >> 31.
uniform  : (x >> 11) * 2^-53 in [0, 1)
normal   : Box-Muller on consecutive pairs (u1, u2):
           r = sqrt(-2 ln(1 - u1)), z0 = r cos(2 pi u2), z1 = r sin(2 pi u2)
Values are produced in float64 and rounded once to float32; the GPU receives
those float32 values and the fp64 oracle receives the same values widened.
Config seeds are 42 + config index (BASELINE.json "configs" order).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start+1 .. start+n of the SplitMix64 stream seeded with `seed`."""
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, low: float = 0.0, high: float = 1.0, dtype=np.float32) -> np.ndarray:
    n = int(np.prod(shape))
    u = (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return (low + (high - low) * u).reshape(shape).astype(dtype)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0, dtype=np.float32) -> np.ndarray:
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = (splitmix64(seed, 2 * m) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log1p(-u1))
    t = 2.0 * np.pi * u2
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return (mean + std * z[:n]).reshape(shape).astype(dtype)
