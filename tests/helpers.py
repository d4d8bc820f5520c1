"""Seeded inputs of the benchmark configurations and comparison helpers."""
from __future__ import annotations

import numpy as np


def c2_input(seed: int = 1) -> np.ndarray:
    """1x128x40x40 ~N(0,1) with 1% of elements (rng.choice, no replacement) x8, fp16-rounded."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((1, 128, 40, 40)).astype(np.float32)
    idx = rng.choice(x.size, size=x.size // 100, replace=False)
    x.reshape(-1)[idx] *= 8.0
    return x.astype(np.float16).astype(np.float32)


def he_weight(rng, oc, ic, k) -> np.ndarray:
    return (rng.standard_normal((oc, ic, k, k)) * np.sqrt(2.0 / (ic * k * k))).astype(np.float32)


def group16_weight(rng, oc, ic, k) -> np.ndarray:
    """He-normal weights whose per-oc int8 scales are equal within 16-row groups.

    The benchmark's "per-16-output-channel-group scales" map onto the
    reference's per-oc scale vector by making every row of a 16-row group
    share its group max: row 16g holds the group's largest |w|.
    """
    w = he_weight(rng, oc, ic, k)
    flat = w.reshape(oc, -1)
    for g in range(0, oc, 16):
        blk = flat[g:g + 16]
        gmax = np.abs(blk).max()
        for r in range(blk.shape[0]):
            i = int(np.argmax(np.abs(blk[r])))
            blk[r, i] = np.sign(blk[r, i] or 1.0) * gmax
    return w


def tol_range(ref: np.ndarray, got: np.ndarray, frac: float) -> tuple[float, float]:
    """(max abs error, allowed) with allowed = frac * output range."""
    rng_ = float(ref.max() - ref.min()) if ref.size else 0.0
    err = float(np.abs(ref.astype(np.float64) - got.astype(np.float64)).max()) if ref.size else 0.0
    return err, frac * max(rng_, 1e-30)


def nchw_to_nhwc(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(a, (0, 2, 3, 1)))


def nhwc_to_nchw(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(a, (0, 3, 1, 2)))
