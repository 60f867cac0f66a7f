"""Deterministic test inputs from integer arithmetic only (splitmix64), so a
fixture needs just its seed: the same float32 bits on every machine.

values: (sum of four 12-bit uniforms - 8190) / 2048, an approximately normal
variable with sd ~1.15, exactly representable in float32.
"""
import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x):
    x = np.asarray(x, np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def det_normal(seed, n):
    idx = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = splitmix64(idx ^ splitmix64(np.uint64(seed)))
    s = np.zeros(n, np.int64)
    for k in range(4):
        s += ((h >> np.uint64(12 * k)) & np.uint64(0xFFF)).astype(np.int64)
    return ((s - 8190).astype(np.float32) / np.float32(2048.0)).astype(np.float32)


class Stream:
    """Successive det_normal blocks from one seed."""

    def __init__(self, seed):
        self.seed = seed
        self.k = 0

    def take(self, n):
        self.k += 1
        return det_normal(self.seed * 1000003 + self.k, n)
