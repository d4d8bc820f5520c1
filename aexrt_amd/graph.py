"""Backend-neutral graph IR with the reference's API shape (src/aexrt/graph.py).

Values are named tensors; constants live in ``Graph.constants``.  Only what
the conv path needs is interpreted here (shape inference for Conv, Sigmoid,
Mul, Add, Split, Concat, MaxPool, Resize, Reshape), but the container itself
accepts any node, like the reference's.
"""
from __future__ import annotations

import copy
import json
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

Shape = Tuple[int, ...]


@dataclass(frozen=True)
class TensorSpec:
    shape: Shape
    dtype: str = "float32"
    layout: str = "contiguous"

    def to_json(self) -> Dict[str, Any]:
        return {"shape": list(self.shape), "dtype": self.dtype, "layout": self.layout}

    @staticmethod
    def from_json(data: Dict[str, Any]) -> "TensorSpec":
        return TensorSpec(tuple(int(v) for v in data["shape"]), data.get("dtype", "float32"),
                          data.get("layout", "contiguous"))


@dataclass
class Node:
    op: str
    name: str
    inputs: List[str]
    outputs: List[str]
    attrs: Dict[str, Any] = field(default_factory=dict)

    def to_json(self) -> Dict[str, Any]:
        return {"op": self.op, "name": self.name, "inputs": self.inputs, "outputs": self.outputs,
                "attrs": self.attrs}

    @staticmethod
    def from_json(data: Dict[str, Any]) -> "Node":
        return Node(data["op"], data["name"], list(data["inputs"]), list(data["outputs"]),
                    dict(data.get("attrs", {})))


class Graph:
    """Named-tensor DAG: inputs, constants, nodes, outputs."""

    def __init__(self, name: str = "graph") -> None:
        self.name = name
        self.metadata: Dict[str, str] = {}
        self.inputs: Dict[str, TensorSpec] = {}
        self.outputs: List[str] = []
        self.constants: Dict[str, np.ndarray] = {}
        self.nodes: List[Node] = []
        self.value_specs: Dict[str, TensorSpec] = {}

    def clone(self) -> "Graph":
        return copy.deepcopy(self)

    def input(self, name: str, spec: TensorSpec) -> "Graph":
        self.inputs[name] = spec
        self.value_specs[name] = spec
        return self

    def const(self, name: str, value: Any, dtype: Optional[str] = None) -> "Graph":
        arr = np.asarray(value, dtype=dtype)
        self.constants[name] = arr
        self.value_specs[name] = TensorSpec(tuple(int(v) for v in arr.shape), str(arr.dtype))
        return self

    def output(self, name: str) -> "Graph":
        if name not in self.outputs:
            self.outputs.append(name)
        return self

    def node(self, op: str, out, *inputs: str, name: Optional[str] = None, **attrs: Any) -> "Graph":
        outs = [out] if isinstance(out, str) else list(out)
        self.nodes.append(Node(op, name or f"{op}_{len(self.nodes)}", list(inputs), outs, dict(attrs)))
        return self

    # builder helpers (graph.py:81-137)
    def add(self, out, a, b): return self.node("Add", out, a, b)
    def mul(self, out, a, b): return self.node("Mul", out, a, b)
    def sigmoid(self, out, x): return self.node("Sigmoid", out, x)
    def reshape(self, out, x, shape: Sequence[int]): return self.node("Reshape", out, x, shape=list(shape))
    def concat(self, out, *xs, axis: int = -1): return self.node("Concat", out, *xs, axis=axis)

    def conv2d(self, out, x, weight, bias=None, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1),
               group: int = 1, name: Optional[str] = None) -> "Graph":
        ins = [x, weight] + ([bias] if bias is not None else [])
        return self.node("Conv", out, *ins, name=name, strides=list(strides), pads=list(pads),
                         dilations=list(dilations), group=int(group))

    def split(self, outs: Sequence[str], x, split: Sequence[int], axis: int = 1) -> "Graph":
        return self.node("Split", list(outs), x, axis=axis, split=list(split))

    def maxpool(self, out, x, kernel: int, stride: int, pad: int) -> "Graph":
        return self.node("MaxPool", out, x, kernel_shape=[kernel, kernel], strides=[stride, stride],
                         pads=[pad, pad, pad, pad], dilations=[1, 1])

    def resize_nearest(self, out, x, scale: int) -> "Graph":
        return self.node("Resize", out, x, mode="nearest", scales=[1, 1, scale, scale])

    def to_json(self) -> Dict[str, Any]:
        return {
            "name": self.name,
            "metadata": dict(self.metadata),
            "inputs": {k: v.to_json() for k, v in self.inputs.items()},
            "outputs": list(self.outputs),
            "constants": {k: v.tolist() for k, v in self.constants.items()},
            "constant_dtypes": {k: str(v.dtype) for k, v in self.constants.items()},
            "nodes": [n.to_json() for n in self.nodes],
        }

    def save_json(self, path: str) -> None:
        with open(path, "w", encoding="utf-8") as f:
            json.dump(self.to_json(), f)

    @staticmethod
    def from_json(data: Dict[str, Any]) -> "Graph":
        g = Graph(data.get("name", "graph"))
        g.metadata = {str(k): str(v) for k, v in data.get("metadata", {}).items()}
        for name, spec in data.get("inputs", {}).items():
            g.input(name, TensorSpec.from_json(spec))
        dtypes = data.get("constant_dtypes", {})
        for name, value in data.get("constants", {}).items():
            g.const(name, value, dtype=dtypes.get(name))
        for n in data.get("nodes", []):
            g.nodes.append(Node.from_json(n))
        for out in data.get("outputs", []):
            g.output(out)
        return g

    @staticmethod
    def load_json(path: str) -> "Graph":
        with open(path, "r", encoding="utf-8") as f:
            return Graph.from_json(json.load(f))


def infer_value_specs(graph: Graph) -> Dict[str, TensorSpec]:
    """Static shapes of every value (the subset of execution.py:253 the conv path uses)."""
    specs: Dict[str, TensorSpec] = dict(graph.value_specs)
    for name, arr in graph.constants.items():
        specs[name] = TensorSpec(tuple(int(v) for v in arr.shape), str(arr.dtype))
    for node in graph.nodes:
        ins = [specs[i].shape for i in node.inputs]
        op = node.op
        if op == "Conv":
            x, w = ins[0], ins[1]
            s = node.attrs.get("strides", [1, 1])
            p = node.attrs.get("pads", [0, 0, 0, 0])
            d = node.attrs.get("dilations", [1, 1])
            oh = (x[2] + p[0] + p[2] - d[0] * (w[2] - 1) - 1) // s[0] + 1
            ow = (x[3] + p[1] + p[3] - d[1] * (w[3] - 1) - 1) // s[1] + 1
            outs = [(x[0], w[0], oh, ow)]
        elif op in ("Sigmoid", "Relu", "Identity"):
            outs = [ins[0]]
        elif op in ("Add", "Mul", "Sub", "Div"):
            outs = [tuple(np.broadcast_shapes(ins[0], ins[1]))]
        elif op == "Split":
            axis = node.attrs.get("axis", 0) % len(ins[0])
            outs = []
            for size in node.attrs["split"]:
                sh = list(ins[0])
                sh[axis] = int(size)
                outs.append(tuple(sh))
        elif op == "Concat":
            axis = node.attrs.get("axis", 0) % len(ins[0])
            sh = list(ins[0])
            sh[axis] = sum(int(s[axis]) for s in ins)
            outs = [tuple(sh)]
        elif op == "MaxPool":
            x = ins[0]
            k = node.attrs["kernel_shape"]
            s = node.attrs.get("strides", k)
            p = node.attrs.get("pads", [0, 0, 0, 0])
            outs = [(x[0], x[1], (x[2] + p[0] + p[2] - k[0]) // s[0] + 1, (x[3] + p[1] + p[3] - k[1]) // s[1] + 1)]
        elif op == "Resize":
            x = ins[0]
            sc = node.attrs.get("scales", [1, 1, 2, 2])
            outs = [(x[0], x[1], int(x[2] * sc[2]), int(x[3] * sc[3]))]
        elif op == "Reshape":
            shape = list(node.attrs["shape"])
            total = int(np.prod(ins[0]))
            if -1 in shape:
                known = int(np.prod([v for v in shape if v != -1]))
                shape[shape.index(-1)] = total // known
            outs = [tuple(int(v) for v in shape)]
        else:
            raise NotImplementedError(f"shape inference for {op}")
        for name, shp in zip(node.outputs, outs):
            specs[name] = TensorSpec(tuple(int(v) for v in shp), "float32")
    return specs
