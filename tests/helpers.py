"""Seeded inputs of the benchmark configurations and comparison helpers."""
from __future__ import annotations

import numpy as np

from aexrt_amd.workloads import c2_input, group16_weight, he_weight  # noqa: F401  (the configurations' generators)


def tol_range(ref: np.ndarray, got: np.ndarray, frac: float) -> tuple[float, float]:
    """(max abs error, allowed) with allowed = frac * output range."""
    rng_ = float(ref.max() - ref.min()) if ref.size else 0.0
    err = float(np.abs(ref.astype(np.float64) - got.astype(np.float64)).max()) if ref.size else 0.0
    return err, frac * max(rng_, 1e-30)


def nchw_to_nhwc(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(a, (0, 2, 3, 1)))


def nhwc_to_nchw(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(a, (0, 3, 1, 2)))
