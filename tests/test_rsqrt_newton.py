"""CPU pin of the RMSNorm factor's device iteration (rsqrt_via_f64, orator_amd/csrc/common.hpp):
two fp64 Newton steps y += y/2 (1 - x y^2) from an fp32 reciprocal-square-root estimate within
one float ulp, then rounded to float, must give (float)(1 / sqrt((double)x)) -- the oracle's
correctly rounded double formula (oracle/orator_oracle.c, RmsNorm) -- so the kernels stay
bit-identical to it.  The estimate is taken one ulp below, at, and one ulp above the float
value, as v_rsq_f32 (1-ulp accurate) may return any of them.  From a start 2^-14 off (where the
quadratic convergence needs both steps) one step is shown to miss, so the comparison can fail."""
from __future__ import annotations

import numpy as np


def _newton(x32: np.ndarray, est32: np.ndarray, steps: int) -> np.ndarray:
    xd = x32.astype(np.longdouble)
    y = est32.astype(np.float64)
    for _ in range(steps):
        # fma(-x*y, y, 1) and fma(y/2, e, y) with one rounding each to double (extended
        # precision intermediates stand in for the fused operations)
        yl = y.astype(np.longdouble)
        e = (1.0 - (xd * yl) * yl).astype(np.float64)
        y = ((0.5 * yl) * e.astype(np.longdouble) + yl).astype(np.float64)
    return y.astype(np.float32)


def _inputs(n: int = 400_000):
    rng = np.random.default_rng(7)
    x = (rng.uniform(1, 2, n) * 2.0 ** rng.integers(-40, 60, n)).astype(np.float32)
    ref = (1.0 / np.sqrt(x.astype(np.float64))).astype(np.float32)
    return x, ref


def test_two_newton_steps_reproduce_the_double_formula():
    x, ref = _inputs()
    for est in (np.nextafter(ref, np.float32(0)), ref, np.nextafter(ref, np.float32(np.inf))):
        assert np.count_nonzero(_newton(x, est, 2) != ref) == 0


def test_the_comparison_detects_a_missing_step():
    x, ref = _inputs()
    coarse = (ref.astype(np.float64) * (1 + 2.0 ** -14)).astype(np.float32)
    assert np.count_nonzero(_newton(x, coarse, 1) != ref) > 0
    assert np.count_nonzero(_newton(x, coarse, 2) != ref) == 0
