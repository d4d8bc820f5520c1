"""Synthetic inputs and weights of the benchmark configurations (seeded, numpy).

* C1: 1x64x80x80 fp32 ~N(0,1); 3x3 s1 p1 64->64, weights ~N(0, sqrt(2/576)), bias ~U(-0.1, 0.1), seed 0.
* C2: 1x128x40x40 ~N(0,1) with 1% of the elements (rng.choice, no replacement) x8, fp16; 1x1
  128->256 with per-16-output-channel-group weight scales, seed 1.
* C3: Bx64x160x160 ~N(0,1) -> 3x3 s2 p1 -> 128x80x80, He-normal weights, seed 2.
* C4: the C2f block (1x1 128->128, split 2x64, two bottlenecks of two 3x3 64->64 with residual,
  concat 4x64 -> 1x1 256->128, SiLU after every conv) at 1x128x40x40, seed 3.
* C5: YOLOv8n-320 (aexrt_amd.yolov8), U(0,1) images, seed 4.

Weights of every config are random (there are no checkpoints); the engine and the tests draw
them from the same generators.
"""
from __future__ import annotations

import numpy as np

from .graph import Graph, TensorSpec


def he_weight(rng: np.random.Generator, oc: int, ic: int, k: int) -> np.ndarray:
    return (rng.standard_normal((oc, ic, k, k)) * np.sqrt(2.0 / (ic * k * k))).astype(np.float32)


def group16_weight(rng: np.random.Generator, oc: int, ic: int, k: int) -> np.ndarray:
    """He-normal weights whose per-oc int8 scales are equal within 16-row groups.

    The configuration's "per-16-output-channel-group scales" map onto the reference's per-oc
    scale vector by making every row of a 16-row group share its group max: each row's largest
    |w| is set to the group's largest |w|.
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


def c1_case():
    """(x, w, b) of C1, seed 0."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 64, 80, 80)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, 64).astype(np.float32)
    return x, w, b


def c2_input(seed: int = 1) -> np.ndarray:
    """1x128x40x40 ~N(0,1) with 1% of elements (rng.choice, no replacement) x8, fp16-rounded."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((1, 128, 40, 40)).astype(np.float32)
    idx = rng.choice(x.size, size=x.size // 100, replace=False)
    x.reshape(-1)[idx] *= 8.0
    return x.astype(np.float16).astype(np.float32)


def c2_case():
    """(x, w, b) of C2: the input above, group-scaled 256x128 1x1 weights, fp16 bias."""
    x = c2_input(1)
    rng = np.random.default_rng(1)
    w = group16_weight(rng, 256, 128, 1)
    b = rng.uniform(-0.1, 0.1, 256).astype(np.float16).astype(np.float32)
    return x, w, b


def c3_case(batch: int):
    """(x, w, b) of C3 at `batch` images (x fp16-rounded), seed 2."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((batch, 64, 160, 160)).astype(np.float32).astype(np.float16).astype(np.float32)
    w = he_weight(rng, 128, 64, 3)
    b = rng.uniform(-0.1, 0.1, 128).astype(np.float16).astype(np.float32)
    return x, w, b


def c2f_block(batch: int = 1, c: int = 128, dim: int = 40, seed: int = 3, shortcut: bool = True) -> Graph:
    """C2f block: 1x1 c->c, split 2x(c/2), two bottlenecks (3x3 pair + residual), concat 4 -> 1x1
    2c->c, every conv followed by SiLU (Conv -> Sigmoid -> Mul, fused by the compiler)."""
    rng = np.random.default_rng(seed)
    g = Graph("c2f")
    g.input("x", TensorSpec((batch, c, dim, dim)))
    k = [0]

    def conv(x, cin, cout, ks):
        k[0] += 1
        n = f"conv{k[0]}"
        g.const(f"{n}.w", he_weight(rng, cout, cin, ks))
        g.const(f"{n}.b", rng.uniform(-0.1, 0.1, cout).astype(np.float32))
        p = ks // 2
        g.conv2d(f"{n}.y", x, f"{n}.w", f"{n}.b", pads=(p, p, p, p), name=n)
        g.sigmoid(f"{n}.s", f"{n}.y")
        g.mul(f"{n}.o", f"{n}.y", f"{n}.s")
        return f"{n}.o"

    h = c // 2
    y = conv("x", c, c, 1)
    g.split(["a", "b"], y, [h, h], axis=1)
    parts = ["a", "b"]
    for i in range(2):
        t = conv(conv(parts[-1], h, h, 3), h, h, 3)
        if shortcut:
            g.add(f"res{i}", parts[-1], t)
            t = f"res{i}"
        parts.append(t)
    g.concat("cat", *parts, axis=1)
    out = conv("cat", 2 * c, c, 1)
    g.output(out)
    return g
