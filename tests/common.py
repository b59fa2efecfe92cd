"""Shared helpers for the tests: the reference's splitmix64 test generator and FNV-1a."""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1


class Rng:
    """The splitmix64 stream of crates/sampling/tests/xcheck.rs:7-16 and crates/cuda/tests/common/mod.rs:100-117."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & M64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def uniform(self, lo: float, hi: float) -> np.float32:
        """crates/cuda/tests/common/mod.rs:110-113: lo + (hi - lo) * ((next >> 40) / 2^24), in f32."""
        lo, hi = np.float32(lo), np.float32(hi)
        return np.float32(lo + np.float32(hi - lo) * np.float32(np.float32(self.next() >> 40) / np.float32(16777216.0)))


def fnv(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h ^= b
        h = (h * 0x100000001B3) & M64
    return h


def splitmix_array(seed: int, n: int) -> np.ndarray:
    """n outputs of the splitmix64 stream, vectorised (same values as Rng(seed).next() n times)."""
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z
