"""Seeded synthetic inputs with a fully specified generator.

The reference draws inputs from std::mt19937 + std::normal_distribution, whose
normal transform is implementation-defined, so its streams cannot be
reproduced bit-for-bit elsewhere.  This module fixes its own:

    word(seed, stream, i) = splitmix64(seed * 0x9E3779B97F4A7C15 ^ stream << 32 ^ i)
    u = ((word >> 11) + 1) * 2**-53                       in (0, 1]
    normal(i) = sqrt(-2 ln u(2i)) * cos(2 pi u(2i+1))      (Box-Muller, fp64)

rounded once to fp32.  Tests and golden fixtures derive every input from
(seed, stream) pairs, so the same tensors can be rebuilt on any host.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _words(seed: int, stream: int, start: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        key = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLDEN
        key ^= np.uint64((stream & 0xFFFFFFFF) << 32)
    idx = np.arange(start, start + n, dtype=np.uint64)
    return _splitmix64(key ^ idx)


def uniform(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """n fp64 uniforms in (0, 1]."""
    w = _words(seed, stream, start, n)
    return ((w >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)


def normal(seed: int, stream: int, shape, scale: float = 1.0, chunk: int = 1 << 22) -> np.ndarray:
    """fp32 array of the given shape, i.i.d. scale * N(0, 1)."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape)) if shape else 1
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        u = uniform(seed, stream, 2 * m, start=2 * s)
        z = np.sqrt(-2.0 * np.log(u[0::2])) * np.cos(2.0 * np.pi * u[1::2])
        out[s:s + m] = (z * scale).astype(np.float32)
    return out.reshape(shape)


def permutation(seed: int, stream: int, n: int) -> np.ndarray:
    """Seeded Fisher-Yates shuffle of 0..n-1 (int64)."""
    u = uniform(seed, stream, max(n - 1, 0))
    p = np.arange(n, dtype=np.int64)
    for i in range(n - 1, 0, -1):
        j = int(u[n - 1 - i] * (i + 1))
        j = min(j, i)
        p[i], p[j] = p[j], p[i]
    return p


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest-even) and widen back to fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, ((u >> 16) | 0x40) << 16, r)
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(x))


# ---------------------------------------------------------------- workloads

def stream_inputs(T: int, d: int, seed: int, scale: float = 1.0, outlier_frac: float = 0.0,
                  outlier_mult: float = 8.0):
    """Q [d], K [T, d], V [T, d]; optionally scale a seeded set of K rows."""
    Q = normal(seed, 1, d, scale)
    K = normal(seed, 2, (T, d), scale)
    V = normal(seed, 3, (T, d), scale)
    n_out = int(outlier_frac * T)
    if n_out:
        rows = permutation(seed, 4, T)[:n_out]
        K[rows] *= np.float32(outlier_mult)
    return Q, K, V


def batch_lengths(B: int = 64, lo: int = 512, hi: int = 32768, seed: int = 70):
    """Per-sequence context lengths ~ U[lo, hi] (seeded): the ragged batch of
    the 64-sequence paged decode workload."""
    u = uniform(seed, 1, B)
    return [int(lo + min(int(x * (hi - lo + 1)), hi - lo)) for x in u]
