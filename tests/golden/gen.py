"""Deterministic synthetic weights for golden vectors and parity tests.

Values come from a splitmix64 integer hash turned into float32 with only
correctly rounded IEEE operations (+, -, *, /, sqrt), so every machine and
numpy version produces the same bits.  No transcendental function and no
library RNG stream is involved.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x):
    x = np.asarray(x, dtype=np.uint64) + _GOLDEN
    z = (x ^ (x >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    """float32 in [0, 1) on a 2^-24 grid."""
    base = np.uint64((seed * 1_000_003 + stream) & 0xFFFFFFFF) << np.uint64(32)
    with np.errstate(over="ignore"):
        h = splitmix64(base + np.arange(n, dtype=np.uint64))
    return (h >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    """Unit-variance bell curve (Irwin-Hall of 4 uniforms), float32."""
    s = uniform(seed, 4 * stream, n) + uniform(seed, 4 * stream + 1, n)
    s = s + uniform(seed, 4 * stream + 2, n) + uniform(seed, 4 * stream + 3, n)
    return (s - np.float32(2.0)) * np.float32(np.sqrt(np.float32(3.0)))


def heavy(seed: int, stream: int, n: int) -> np.ndarray:
    """Heavy-tailed unit-ish variance draws: normal scaled by 1 / sqrt(chi-like)."""
    z = normal(seed, 3 * stream, n)
    a = normal(seed, 3 * stream + 1, n)
    b = normal(seed, 3 * stream + 2, n)
    chi = (a * a + b * b) * np.float32(0.5) + np.float32(0.05)
    return z / np.sqrt(chi) * np.float32(0.5)


def correlated_models(seed: int, lengths, base_std=0.02, delta_std=0.002, delta_growth=True):
    """Base ~ heavy-tailed * base_std, model i = base + delta_std*(i+1) * normal.

    ``lengths`` gives each model's flat length (the base is drawn for the
    longest one).  Returns a list of float32 arrays.
    """
    nmax = max(lengths)
    w0 = heavy(seed, 0, nmax) * np.float32(base_std)
    out = []
    for i, L in enumerate(lengths):
        ds = np.float32(delta_std * ((i + 1) if delta_growth else 1))
        out.append((w0[:L] + normal(seed, 10 + i, L) * ds).astype(np.float32))
    return out
