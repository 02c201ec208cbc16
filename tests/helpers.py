"""Shared test helpers: seeded inputs and the error measures the tolerances use."""
from __future__ import annotations

import numpy as np


class SplitMix64:
    """Seeded generator of our own (SplitMix64 + Box-Muller), so inputs do not depend on
    a library's distribution code."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed)

    def _next(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            idx = np.arange(1, n + 1, dtype=np.uint64)
            z = self.state + idx * np.uint64(0x9E3779B97F4A7C15)
            self.state = self.state + np.uint64(n) * np.uint64(0x9E3779B97F4A7C15)
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        return z

    def uniform(self, n: int) -> np.ndarray:
        """n doubles in (0, 1)."""
        return ((self._next(n) >> np.uint64(11)).astype(np.float64) + 0.5) / float(1 << 53)

    def normal(self, shape, scale: float = 1.0) -> np.ndarray:
        n = int(np.prod(shape))
        m = (n + 1) // 2
        u1, u2 = self.uniform(m), self.uniform(m)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
        return (z * scale).astype(np.float32).reshape(shape)


def rel_err(got, ref, floor):
    """Reference convention |g - r| / max(|r|, floor) (test/unit/model/test_asr_gemm.cc:368)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor)))
