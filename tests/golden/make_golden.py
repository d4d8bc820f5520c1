"""Writes the golden vectors under tests/golden/ (run from the repo root).

Each fixture restates the expected value of one of the reference's own
known-answer tests, computed exactly as that test defines it:

* winograd_f2x2_kat.npz -- tests/test_engine_fp16_winograd_plan.py:76-144:
  32x32 3x3 weights arange(32*32*9)/4096, fp16-rounded, transformed with
  U = G g G^T via numpy.einsum("ak,oikl,bl->oiab", optimize=True), stored as
  fp16 (layout 3) and fp32 (layout 5).
* conv1x1_oc8_kat.npz -- tests/test_engine_fp16_1x1_plan.py:27-73: 64x64
  1x1 weights arange(64*64)/1024, packed [oc/8][ic][8] as fp16 (layout 4).

The reference package itself is not imported; only these definitions are
reproduced.  Inputs are regenerable from the formulas, so only expected
outputs are stored.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
G = np.asarray(((1.0, 0.0, 0.0), (0.5, 0.5, 0.5), (0.5, -0.5, 0.5), (0.0, 0.0, 1.0)), dtype=np.float32)


def winograd_kat_weights() -> np.ndarray:
    return (np.arange(32 * 32 * 9, dtype=np.float32).reshape(32, 32, 3, 3) / 4096.0)


def conv1x1_kat_weights() -> np.ndarray:
    return (np.arange(64 * 64, dtype=np.float32) / 1024.0).reshape(64, 64, 1, 1)


def main() -> None:
    w = winograd_kat_weights()
    q = w.astype("<f2").astype(np.float32)
    u = np.einsum("ak,oikl,bl->oiab", G, q, G, optimize=True)
    np.savez_compressed(HERE / "winograd_f2x2_kat.npz",
                        expected_f16_bits=u.astype("<f2").view(np.uint16),
                        expected_f32=u.astype("<f4"))
    w1 = conv1x1_kat_weights()
    exp = w1.reshape(8, 8, 64).transpose(0, 2, 1).astype("<f2")
    np.savez_compressed(HERE / "conv1x1_oc8_kat.npz", expected_f16_bits=exp.view(np.uint16))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
