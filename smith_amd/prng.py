"""Seeded inputs: SplitMix64 -> uniform (0, 1] -> Box-Muller.

The reference has no seeding (src/tensor.js:116-146 draws Math.random()).
This generator keeps randn's structure -- pairs (u1, u2) -> r*cos(theta),
r*sin(theta) with r = sqrt(-2 ln u1), theta = 2*pi*u2, in f64, stored to f32
(src/tensor.js:129-145) -- with a reproducible uniform source, so every test
and benchmark input is a function of (seed, shape, mean, std).
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed, start, count):
    """Outputs start .. start+count-1 of the SplitMix64 stream seeded with seed."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed, start, count):
    """(0, 1] doubles: ((x >> 11) + 1) * 2^-53."""
    x = splitmix64(seed, start, count)
    return ((x >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)


def randn(shape, seed, std=1.0, mean=0.0):
    """f32 normal samples of the given shape, Box-Muller pairs in f64."""
    shape = tuple(int(s) for s in shape)
    n = int(np.prod(shape)) if shape else 1
    out = np.empty(n, dtype=np.float32)
    npairs = (n + 1) // 2
    for p0 in range(0, npairs, _CHUNK):
        cnt = min(_CHUNK, npairs - p0)
        u = uniform(seed, 2 * p0, 2 * cnt)
        u1, u2 = u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        th = 2.0 * np.pi * u2
        v = np.empty(2 * cnt, dtype=np.float64)
        v[0::2] = r * np.cos(th)
        v[1::2] = r * np.sin(th)
        lo = 2 * p0
        hi = min(n, lo + 2 * cnt)
        out[lo:hi] = (v[: hi - lo] * std + mean).astype(np.float32)
    return out.reshape(shape)


def randint(n, high, seed):
    """n integers in [0, high) (token ids for synthetic prompts)."""
    x = splitmix64(seed, 0, n)
    return (x % np.uint64(high)).astype(np.int64)
