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


def check_fp32(got, ref, tol=1e-4, label="", truth=None, floor3_tol=None, truth_mult=2.0):
    """fp32-mode parity gate.  Always: rel_err(floor 0.05) <= tol.  At the reference's floor
    1e-3 (test/unit/model/test_asr_gemm.cc:368): rel_err(floor 1e-3) <= floor3_tol (tol if
    not given); where fp32 summation over long rows cannot meet that against the oracle (an
    output near 0 is a cancellation of terms ~1000x larger), a test passes `truth` (fp64) and
    the device must be about as close to the exact value as the oracle is: rel_err(got, truth,
    1e-3) <= max(floor3_tol, truth_mult * rel_err(ref, truth, 1e-3)), truth_mult 2 unless a
    test states why its formula is less exact than the oracle's.  Every figure is printed (and
    appended to $ORATOR_PARITY_LOG when set)."""
    import json
    import os
    label = label or os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    e05 = rel_err(got, ref, 0.05)
    e3 = rel_err(got, ref, 1e-3)
    t3 = tol if floor3_tol is None else floor3_tol
    rec = {"test": label, "floor_0.05": e05, "floor_1e-3": e3, "tol": tol, "tol_1e-3": t3}
    ok3 = e3 <= t3
    if not ok3 and truth is not None:
        eo = rel_err(ref, truth, 1e-3)
        eg = rel_err(got, truth, 1e-3)
        rec.update({"oracle_vs_fp64_1e-3": eo, "device_vs_fp64_1e-3": eg})
        ok3 = eg <= max(t3, truth_mult * eo)
    print("[parity]", json.dumps(rec), flush=True)
    path = os.environ.get("ORATOR_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert e05 <= tol, rec
    assert ok3, rec
