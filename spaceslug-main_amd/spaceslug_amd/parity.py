"""Numerical parity report with the reference's metric (python/spaceslug/parity.py:6-16).

error_i = |actual_i - expected_i| / max(1, |expected_i|); status "pass" when every
error_i <= tolerance. Same keys as the reference's report, plus max_abs_error and
normwise_error (||a - e||_2 / ||e||_2), computed with numpy instead of a Python loop.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np


def compare_float_arrays(actual: Sequence[float] | np.ndarray, expected: Sequence[float] | np.ndarray, *,
                         tolerance: float = 1e-3) -> dict:
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    if a.size != e.size:
        raise ValueError("parity arrays must have equal length")
    diff = np.abs(a - e)
    err = diff / np.maximum(1.0, np.abs(e))
    bad = ~(err <= tolerance)  # NaN counts as bad
    first_bad = int(np.argmax(bad)) if bad.any() else None
    maximum = float(np.nanmax(np.where(np.isnan(err), np.inf, err))) if err.size else 0.0
    norm_e = float(np.linalg.norm(e)) if e.size else 0.0
    normwise = float(np.linalg.norm(a - e)) / max(norm_e, 1e-300) if e.size else 0.0
    return {"status": "pass" if first_bad is None else "fail", "tolerance": tolerance,
            "max_relative_error": maximum, "first_bad_index": first_bad, "count": int(a.size),
            "max_abs_error": float(diff.max()) if diff.size else 0.0, "normwise_error": normwise}
