"""SplitMix64 as kapel-ref/src/rng.rs:12-29 (scalar; for the test fixtures that
the reference's own tests build from it)."""

MASK = (1 << 64) - 1


class Rng:
    def __init__(self, seed):
        self.state = seed & MASK

    def next_u64(self):
        self.state = (self.state + 0x9E3779B97F4A7C15) & MASK
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        return z ^ (z >> 31)

    def uniform(self, lo, hi):
        unit = (self.next_u64() >> 11) / float(1 << 53)
        return lo + (hi - lo) * unit


def lcg_bytes(seed):
    """The byte generator of kapel-cpu/src/quantized.rs:1033-1039."""
    state = seed & MASK

    def nxt():
        nonlocal state
        state = (state * 6364136223846793005 + 1442695040888963407) & MASK
        return (state >> 33) & 0xFF

    return nxt
