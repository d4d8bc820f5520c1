"""Whole-network CPU oracle -- TEST INFRASTRUCTURE (see oracle/__init__.py).

Evaluates a Graph with the W8A8 chain on the convs named int8 and fp16
direct convolution on the rest, storing every intermediate tensor as fp16
like the device path (the network output stays fp32).  Each int8 conv is
the reference chain on the fp16-stored input: per-tensor amax over the whole
tensor (all images), RNE quantization with 127/amax, exact int32
accumulation, dequant float(acc)*amax/127*w_scale + bias, SiLU -- or, for
an input of fewer than 4096 elements, the reference's dynamic fallback
(per position and 4-channel group scales computed in the conv).
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional

import numpy as np

from . import (amax, amax_slots, conv_desc, conv_int8_acc, conv_int8_dynamic, conv_int8_epilogue, conv_int8_pg,
               cpu_conv2d, maxpool, quant_pack, quantize, resize_nearest, round_f16, weight_quant)

# The reference prequantizes (amax + pack) only inputs of at least this many
# elements (RT:21478-21479); smaller int8 inputs take the dynamic kernel.
PREQUANT_MIN_ELEMENTS = 4096


def _silu_map(graph):
    consumers = {}
    for i, n in enumerate(graph.nodes):
        for v in n.inputs:
            consumers.setdefault(v, []).append(i)
    out = {}
    for i, n in enumerate(graph.nodes):
        if n.op != "Conv":
            continue
        y = n.outputs[0]
        users = consumers.get(y, [])
        if len(users) != 2:
            continue
        sig = [u for u in users if graph.nodes[u].op == "Sigmoid"]
        mul = [u for u in users if graph.nodes[u].op == "Mul"]
        if len(sig) == 1 and len(mul) == 1:
            out[i] = (sig[0], mul[0])
    return out


def conv_layer(x: np.ndarray, w: np.ndarray, b: np.ndarray, attrs: dict, *, int8: bool, silu: bool,
               threads: int = 1, pg16: bool = False) -> np.ndarray:
    """One conv of the network on an fp16-valued input, fp32 result (unrounded).

    pg16: the reference's per-group path (plan flag 16): strip amax
    (RT:3219-3259), per-group pack (RT:3314-3346), pg16 conv (RT:4770-4923).
    """
    n, c, h, wd = x.shape
    k = int(w.shape[2])
    s = int(attrs.get("strides", [1, 1])[0])
    p = int(attrs.get("pads", [0, 0, 0, 0])[0])
    desc = conv_desc(n, c, h, wd, int(w.shape[0]), k, s, p)
    bias = round_f16(b)
    if int8 and x.size < PREQUANT_MIN_ELEMENTS:
        # RT:21478-21479: an input of fewer than 4096 elements is not
        # prequantized; the conv quantizes per (position, 4 channels) itself
        # (RT:2952-3115), pg16 or not
        qw, ws = weight_quant(w, fp16_round=True)
        return conv_int8_dynamic(x, qw, desc, ws, bias, silu)
    if int8 and pg16:
        slots = amax_slots(x)
        packed = quant_pack(x, slots, per_group=True)
        qw, ws = weight_quant(w, fp16_round=True)
        return conv_int8_pg(packed, qw, desc, slots, ws, bias, silu)
    if int8:
        a = amax(x)
        qa = quantize(x, a)
        qw, ws = weight_quant(w, fp16_round=True)
        acc = conv_int8_acc(qa, qw, desc, threads=threads)
        return conv_int8_epilogue(acc, a, ws, bias, silu)
    return cpu_conv2d(x, round_f16(w), bias, desc, silu, threads=threads)


def run_graph(graph, image: np.ndarray, int8_convs: Optional[Iterable[str]] = None, threads: int = 1,
              keep: bool = False) -> Dict[str, np.ndarray]:
    """Runs the graph; returns {output name: array} (every value when keep=True)."""
    int8 = set(int8_convs or ())
    silu = _silu_map(graph)
    skip = set()
    for a, b in silu.values():
        skip.update((a, b))
    vals: Dict[str, np.ndarray] = {name: np.asarray(image, np.float32) for name in graph.inputs}
    for name, arr in graph.constants.items():
        vals[name] = np.asarray(arr, np.float32)
    out_name = graph.outputs[0]
    for i, node in enumerate(graph.nodes):
        if i in skip:
            continue
        op = node.op
        ins = [vals[v] for v in node.inputs]
        if op == "Conv":
            x = ins[0]
            if node.inputs[0] in graph.inputs:
                x = round_f16(x)
            is_silu = i in silu
            y = conv_layer(x, ins[1], ins[2] if len(ins) > 2 else np.zeros(ins[1].shape[0], np.float32),
                           node.attrs, int8=node.name in int8, silu=is_silu, threads=threads)
            dst = graph.nodes[silu[i][1]].outputs[0] if is_silu else node.outputs[0]
            vals[dst] = y if dst == out_name else round_f16(y)
            continue
        if op == "Add":
            y = round_f16(ins[0] + ins[1])
        elif op == "Split":
            axis = node.attrs.get("axis", 0)
            bounds = np.cumsum(node.attrs["split"])[:-1]
            for name, part in zip(node.outputs, np.split(ins[0], bounds, axis=axis)):
                vals[name] = np.ascontiguousarray(part)
            continue
        elif op == "Concat":
            y = np.concatenate(ins, axis=node.attrs.get("axis", 0))
        elif op == "MaxPool":
            k = node.attrs["kernel_shape"][0]
            y = maxpool(ins[0], k, node.attrs.get("strides", [k])[0], node.attrs.get("pads", [0])[0])
        elif op == "Resize":
            sc = node.attrs.get("scales", [1, 1, 2, 2])
            y = resize_nearest(ins[0], int(ins[0].shape[2] * sc[2]), int(ins[0].shape[3] * sc[3]))
        elif op == "Reshape":
            y = ins[0].reshape(node.attrs["shape"])
        elif op == "Sigmoid":
            y = round_f16(1.0 / (1.0 + np.exp(-ins[0])))
        elif op == "Mul":
            y = round_f16(ins[0] * ins[1])
        else:
            raise NotImplementedError(op)
        vals[node.outputs[0]] = y
    if keep:
        return vals
    return {out_name: vals[out_name]}
