"""YOLOv8n (width 0.25, depth 0.33, 80 classes) as a Graph, random He init.

Topology of the standard yolov8n model: CSP backbone (Conv s2 stages, C2f
blocks, SPPF), PAN neck (upsample + concat + C2f, Conv s2 + concat + C2f) and
the decoupled Detect head (per level: box branch 3x3-3x3-1x1 to 4*16 DFL
bins, class branch 3x3-3x3-1x1 to 80 logits).  Every Conv+BN+SiLU appears as
an ONNX-style Conv -> Sigmoid -> Mul with BN folded into the conv (identity
BN), which the compiler fuses into CONV_SILU.  ``output0`` is the raw head
tensor [B, 144, anchors] (box bins then class logits), before DFL decode.

63 convolutions, 3.15 M parameters, 2.19 GOP per 320x320 image.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .graph import Graph, TensorSpec

NUM_CLASSES = 80
REG_MAX = 16


@dataclass
class _Builder:
    graph: Graph
    rng: np.random.Generator
    counter: int = 0
    convs: list = field(default_factory=list)  # (name, stage tag)

    def _name(self, base: str) -> str:
        self.counter += 1
        return f"{base}_{self.counter}"

    def conv(self, x: str, cin: int, cout: int, k: int, s: int, tag: str, act: bool = True) -> str:
        g = self.graph
        name = self._name(f"{tag}.conv")
        w = (self.rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
        b = self.rng.uniform(-0.1, 0.1, cout).astype(np.float32)
        g.const(f"{name}.w", w)
        g.const(f"{name}.b", b)
        p = k // 2
        out = f"{name}.y"
        g.conv2d(out, x, f"{name}.w", f"{name}.b", strides=(s, s), pads=(p, p, p, p), name=name)
        self.convs.append((name, tag))
        if not act:
            return out
        g.sigmoid(f"{name}.sig", out)
        g.mul(f"{name}.silu", out, f"{name}.sig")
        return f"{name}.silu"

    def bottleneck(self, x: str, c: int, shortcut: bool, tag: str) -> str:
        y = self.conv(x, c, c, 3, 1, tag)
        y = self.conv(y, c, c, 3, 1, tag)
        if shortcut:
            out = self._name(f"{tag}.add")
            self.graph.add(out, x, y)
            return out
        return y

    def c2f(self, x: str, c1: int, c2: int, n: int, shortcut: bool, tag: str) -> str:
        c = c2 // 2
        y = self.conv(x, c1, 2 * c, 1, 1, tag)
        a, b = self._name(f"{tag}.split0"), self._name(f"{tag}.split1")
        self.graph.split([a, b], y, [c, c], axis=1)
        parts = [a, b]
        for _ in range(n):
            parts.append(self.bottleneck(parts[-1], c, shortcut, tag))
        cat = self._name(f"{tag}.cat")
        self.graph.concat(cat, *parts, axis=1)
        return self.conv(cat, (2 + n) * c, c2, 1, 1, tag)

    def sppf(self, x: str, c1: int, c2: int, tag: str) -> str:
        c_ = c1 // 2
        y = [self.conv(x, c1, c_, 1, 1, tag)]
        for _ in range(3):
            out = self._name(f"{tag}.pool")
            self.graph.maxpool(out, y[-1], 5, 1, 2)
            y.append(out)
        cat = self._name(f"{tag}.cat")
        self.graph.concat(cat, *y, axis=1)
        return self.conv(cat, 4 * c_, c2, 1, 1, tag)

    def upsample(self, x: str) -> str:
        out = self._name("neck.up")
        self.graph.resize_nearest(out, x, 2)
        return out

    def cat(self, *xs: str) -> str:
        out = self._name("neck.cat")
        self.graph.concat(out, *xs, axis=1)
        return out


def build_yolov8n(batch: int = 1, imgsz: int = 320, seed: int = 4, num_classes: int = NUM_CLASSES) -> Graph:
    """YOLOv8n graph with seeded random He-normal weights and U(-0.1, 0.1) biases."""
    g = Graph("yolov8n")
    g.metadata["model"] = "yolov8n"
    g.input("images", TensorSpec((batch, 3, imgsz, imgsz), "float32"))
    B = _Builder(g, np.random.default_rng(seed))
    # backbone
    x = B.conv("images", 3, 16, 3, 2, "stem")
    x = B.conv(x, 16, 32, 3, 2, "b1")
    x = B.c2f(x, 32, 32, 1, True, "b2")
    x = B.conv(x, 32, 64, 3, 2, "b3")
    p3 = B.c2f(x, 64, 64, 2, True, "b4")
    x = B.conv(p3, 64, 128, 3, 2, "b5")
    p4 = B.c2f(x, 128, 128, 2, True, "b6")
    x = B.conv(p4, 128, 256, 3, 2, "b7")
    x = B.c2f(x, 256, 256, 1, True, "b8")
    p5 = B.sppf(x, 256, 256, "b9")
    # neck (PAN)
    x = B.cat(B.upsample(p5), p4)
    n12 = B.c2f(x, 384, 128, 1, False, "n12")
    x = B.cat(B.upsample(n12), p3)
    n15 = B.c2f(x, 192, 64, 1, False, "n15")
    x = B.cat(B.conv(n15, 64, 64, 3, 2, "n16"), n12)
    n18 = B.c2f(x, 192, 128, 1, False, "n18")
    x = B.cat(B.conv(n18, 128, 128, 3, 2, "n19"), p5)
    n21 = B.c2f(x, 384, 256, 1, False, "n21")
    # detect head
    c2 = max(16, 64 // 4, REG_MAX * 4)
    c3 = max(64, min(num_classes, 100))
    levels = []
    for i, (feat, ch) in enumerate(((n15, 64), (n18, 128), (n21, 256))):
        bx = B.conv(feat, ch, c2, 3, 1, f"head{i}.box")
        bx = B.conv(bx, c2, c2, 3, 1, f"head{i}.box")
        bx = B.conv(bx, c2, 4 * REG_MAX, 1, 1, f"head{i}.box", act=False)
        cl = B.conv(feat, ch, c3, 3, 1, f"head{i}.cls")
        cl = B.conv(cl, c3, c3, 3, 1, f"head{i}.cls")
        cl = B.conv(cl, c3, num_classes, 1, 1, f"head{i}.cls", act=False)
        cat = f"head{i}.cat"
        g.concat(cat, bx, cl, axis=1)
        hw = (imgsz // (8 << i)) ** 2
        flat = f"head{i}.flat"
        g.reshape(flat, cat, (batch, 4 * REG_MAX + num_classes, hw))
        levels.append(flat)
    g.concat("output0", *levels, axis=2)
    g.output("output0")
    g.metadata["int8_convs"] = ",".join(n for n, t in B.convs if not (t.startswith("head") or t == "stem"))
    return g


def conv_gops(graph: Graph) -> float:
    """Direct-convolution work (2*MACs) of all convs in GOP."""
    from .graph import infer_value_specs

    specs = infer_value_specs(graph)
    total = 0
    for n in graph.nodes:
        if n.op != "Conv":
            continue
        w = specs[n.inputs[1]].shape
        y = specs[n.outputs[0]].shape
        total += 2 * y[0] * y[1] * y[2] * y[3] * w[1] * w[2] * w[3]
    return total / 1e9
