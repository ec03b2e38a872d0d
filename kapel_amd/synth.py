"""Seeded synthetic inputs: SplitMix64 (as kapel-ref/src/rng.rs:12-18) and a
Box-Muller transform for N(0, sigma) (the reference has no normal generator;
this one is this library's).  Vectorized: value i of seed s comes from the
(i + 1)-th output of SplitMix64(s), so any slice can be made independently.
"""
import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, start, count):
    """Outputs start+1 .. start+count of SplitMix64(seed), as uint64."""
    with np.errstate(over="ignore"):
        n = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + n * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def uniform(seed, count, start=0):
    """Uniform in [0, 1): the top 53 bits (rng.rs:20-24)."""
    return (splitmix64(seed, start, count) >> np.uint64(11)).astype(np.float64) / float(1 << 53)


def normal(seed, count, sigma=1.0, chunk=1 << 24):
    """count values ~ N(0, sigma) as float32: pairs (u1, u2) of uniforms,
    r = sqrt(-2 ln(1 - u1)), r cos(2 pi u2) and r sin(2 pi u2)."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, chunk):
        p = min(chunk, pairs - p0)
        u = uniform(seed, 2 * p, start=2 * p0).reshape(p, 2)
        r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
        theta = 2.0 * np.pi * u[:, 1]
        z = np.empty((p, 2))
        z[:, 0] = r * np.cos(theta)
        z[:, 1] = r * np.sin(theta)
        z = z.ravel() * sigma
        lo = 2 * p0
        hi = min(count, lo + 2 * p)
        out[lo:hi] = z[: hi - lo]
    return out
